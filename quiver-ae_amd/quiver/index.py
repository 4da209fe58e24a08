"""NumPy interface with the reference's API (python/quiver/index.py:27-264).

``IndexQuiver(index_dir, ...).search(queries, topk, ef_search=...)`` returns
``(ids int32[n, topk], distances float32[n, topk])``.  By default the search
runs in-process through libquiver_hip's C ABI on the GPU; when ``binary`` (or
``QUIVER_BINARY``) names an engine executable, the call shells out to it with
the reference's command line and reads its result files, exactly as the
reference binding does.
"""
from __future__ import annotations

import ctypes as C
import os
import shutil
import struct
import subprocess
import tempfile
from pathlib import Path
from typing import Mapping, Sequence

import numpy as np
import numpy.typing as npt

from . import _lib
from ._lib import QuiverError

_DATA_TYPES = {
    "float": (np.dtype("<f4"), ".fbin"),
    "float32": (np.dtype("<f4"), ".fbin"),
    "uint8": (np.dtype("u1"), ".u8bin"),
    "int8": (np.dtype("i1"), ".i8bin"),
}


class IndexQuiver:
    """Search a Quiver index with NumPy arrays.

    Argument meaning, defaults and errors follow the reference binding.  The
    in-process engine keeps the graph, vectors and PQ codes resident in GPU
    memory (the heap memory backend); SSD options are accepted for
    compatibility but the SPDK backend is not part of this library, so a search
    with SSDs configured raises ``QuiverError`` unless an external ``binary``
    is used.
    """

    def __init__(
        self,
        index_dir: str | os.PathLike[str],
        *,
        data_type: str = "float32",
        ssds: Sequence[str] | None = None,
        ssd_list_file: str | os.PathLike[str] | None = None,
        spdk_base_lba: int | None = None,
        binary: str | os.PathLike[str] | None = None,
        memory_backend: str = "heap",
        num_blocks: int = 756,
        queries_per_block: int = 1,
        pipe_width: int = 2,
        poll_threads: int = 6,
        runners_per_ssd: int = 1,
        env: Mapping[str, str] | None = None,
        device: int = 0,
        graph_placement: str = "hbm",
        search_kernel: str = "auto",
    ) -> None:
        self.index_dir = Path(index_dir).expanduser().resolve()
        if not self.index_dir.is_dir():
            raise ValueError(f"index_dir is not a directory: {self.index_dir}")

        normalized_type = data_type.lower()
        if normalized_type not in _DATA_TYPES:
            raise ValueError("data_type must be float32, float, uint8, or int8")
        self.data_type = "float" if normalized_type == "float32" else normalized_type
        self._numpy_dtype, self._query_suffix = _DATA_TYPES[normalized_type]

        if ssds and ssd_list_file:
            raise ValueError("pass either ssds or ssd_list_file, not both")
        self.ssds = tuple(str(ssd).strip() for ssd in (ssds or ()))
        if any(not ssd for ssd in self.ssds):
            raise ValueError("SSD PCI addresses must not be empty")
        self.ssd_list_file = (
            Path(ssd_list_file).expanduser().resolve() if ssd_list_file else None
        )
        if self.ssd_list_file and not self.ssd_list_file.is_file():
            raise ValueError(f"ssd_list_file does not exist: {self.ssd_list_file}")
        if spdk_base_lba is not None and spdk_base_lba < 0:
            raise ValueError("spdk_base_lba must be non-negative")
        self.spdk_base_lba = spdk_base_lba

        if memory_backend not in {"heap", "mmap"}:
            raise ValueError("memory_backend must be heap or mmap")
        self.memory_backend = memory_backend
        if graph_placement not in {"hbm", "host"}:
            raise ValueError("graph_placement must be hbm or host")
        self.graph_placement = graph_placement
        if search_kernel not in _lib.KERNEL_NAMES:
            raise ValueError("search_kernel must be auto, lut or shared-pivots")
        self.search_kernel = search_kernel
        self.binary = self._find_binary(binary)
        self.num_blocks = self._positive(num_blocks, "num_blocks")
        self.queries_per_block = self._positive(queries_per_block, "queries_per_block")
        self.pipe_width = self._positive(pipe_width, "pipe_width")
        self.poll_threads = self._positive(poll_threads, "poll_threads")
        self.runners_per_ssd = self._positive(runners_per_ssd, "runners_per_ssd")
        self.env = dict(env or {})
        self.device = int(device)
        self._handle: C.c_void_p | None = None
        self.last_report: dict | None = None
        if self.binary is None:
            _lib.load()

    @property
    def num_ssds(self) -> int:
        if self.ssds:
            return len(self.ssds)
        if not self.ssd_list_file:
            return 0
        return len(
            [
                line
                for line in self.ssd_list_file.read_text().splitlines()
                if line.strip() and not line.lstrip().startswith("#")
            ]
        )

    def search(
        self,
        queries: npt.ArrayLike,
        topk: int = 10,
        *,
        ef_search: int = 50,
        early_exit_policy: str = "gpruning",
        timeout: float | None = None,
        extra_args: Sequence[str] = (),
    ) -> tuple[npt.NDArray[np.int32], npt.NDArray[np.float32]]:
        """Return ``(ids, distances)`` with shape ``(len(queries), topk)``."""
        topk = self._positive(topk, "topk")
        ef_search = self._positive(ef_search, "ef_search")
        if early_exit_policy not in {"gpruning", "none"}:
            raise ValueError("early_exit_policy must be gpruning or none")
        if timeout is not None and timeout <= 0:
            raise ValueError("timeout must be positive")

        array = np.asarray(queries)
        if array.ndim == 1:
            array = array.reshape(1, -1)
        if array.ndim != 2 or array.shape[0] == 0 or array.shape[1] == 0:
            raise ValueError("queries must be a non-empty 1D or 2D array")
        array = np.ascontiguousarray(array, dtype=self._numpy_dtype)

        if self.binary is not None:
            return self._search_subprocess(array, topk, ef_search, early_exit_policy, timeout, extra_args)
        return self._search_inprocess(array, topk, ef_search, early_exit_policy, timeout, extra_args)

    # ---- in-process engine (C ABI) ---------------------------------------
    def _open(self) -> C.c_void_p:
        if self._handle is None:
            lib = _lib.load()
            h = C.c_void_p()
            _lib.check(
                lib.qv_index_open_ex(
                    str(self.index_dir).encode(),
                    self.data_type.encode(),
                    self.memory_backend.encode(),
                    None,
                    self.device,
                    _lib.QV_GRAPH_HOST if self.graph_placement == "host" else _lib.QV_GRAPH_HBM,
                    C.byref(h),
                )
            )
            self._handle = h
        return self._handle

    def info(self) -> dict:
        info = _lib.IndexInfo()
        _lib.check(_lib.load().qv_index_get_info(self._open(), C.byref(info)))
        return {name: getattr(info, name) for name, _ in info._fields_}

    def _search_inprocess(self, array, topk, ef_search, early_exit_policy, timeout, extra_args):
        extra = [str(x) for x in extra_args]
        skip_nav = "--skip-nav" in extra
        extra = [x for x in extra if x != "--skip-nav"]
        if extra:
            raise QuiverError("extra_args other than --skip-nav need an external quiver_search binary")
        if self.num_ssds:
            raise QuiverError("This binary was built without SPDK support")
        handle = self._open()
        q = np.ascontiguousarray(array, dtype=np.float32)
        n, d = q.shape
        ids = np.empty((n, topk), dtype=np.int32)
        dists = np.empty((n, topk), dtype=np.float32)
        found = np.empty((n,), dtype=np.int32)
        opts = _lib.default_search_opts()
        opts.num_blocks = self.num_blocks
        opts.queries_per_block = self.queries_per_block
        opts.pipe_width = self.pipe_width
        opts.early_exit = _lib.QV_EXIT_GPRUNING if early_exit_policy == "gpruning" else _lib.QV_EXIT_NONE
        env = {**os.environ, **self.env}
        if "QUIVER_PREFEED" in env:
            opts.prefeed = int(env["QUIVER_PREFEED"])
        if "QUIVER_ADMIT_MIN_BATCH" in env:
            opts.admit_min_batch = max(1, int(env["QUIVER_ADMIT_MIN_BATCH"]))
        opts.timeout_s = float(timeout) if timeout is not None else 0.0
        opts.skip_nav = 1 if skip_nav else 0
        opts.kernel = _lib.KERNEL_NAMES[self.search_kernel]
        rep = _lib.SearchReport()
        rc = _lib.load().qv_search(
            handle, q.ctypes.data, n, d, topk, ef_search, C.byref(opts),
            ids.ctypes.data, dists.ctypes.data, found.ctypes.data, C.byref(rep),
        )
        if rc == _lib.QV_ETIMEDOUT:
            raise QuiverError(f"quiver_search exceeded the {timeout:g} second timeout")
        _lib.check(rc)
        self.last_report = rep.as_dict()
        return ids, dists

    def load_nav(self, nav_dir: str | os.PathLike[str]) -> None:
        """Load (or replace) the navigation graph that picks each query's entry
        node (nav_index, nav_index.data, map.txt).  An index directory holding
        nav_index or nav/nav_index gets its graph at open without this call."""
        _lib.check(_lib.load().qv_index_load_nav(self._open(), str(nav_dir).encode()))

    def close(self) -> None:
        if self._handle is not None:
            _lib.load().qv_index_close(self._handle)
            self._handle = None

    def __enter__(self) -> "IndexQuiver":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    # ---- external engine (reference command line) ------------------------
    def _search_subprocess(self, array, topk, ef_search, early_exit_policy, timeout, extra_args):
        with tempfile.TemporaryDirectory(prefix="quiver-python-") as temp_dir:
            work = Path(temp_dir)
            query_path = work / f"queries{self._query_suffix}"
            result_prefix = work / "result"
            self._write_bin(query_path, array)
            ssd_list = self._materialize_ssd_list(work)

            command = [
                str(self.binary),
                "--index-dir", str(self.index_dir),
                "--query", str(query_path),
                "--data-type", self.data_type,
                "--topk", str(topk),
                "--ef-search", str(ef_search),
                "--repeat", "1",
                "--num-blocks", str(self.num_blocks),
                "--queries-per-block", str(self.queries_per_block),
                "--pipe-width", str(self.pipe_width),
                "--poll-threads", str(self.poll_threads),
                "--runners-per-ssd", str(self.runners_per_ssd),
                "--memory-backend", self.memory_backend,
                "--early-exit-policy", early_exit_policy,
                "--result-prefix", str(result_prefix),
            ]
            if ssd_list is not None:
                command.extend(["--ssd-list-file", str(ssd_list)])
            command.extend(str(arg) for arg in extra_args)

            process_env = os.environ.copy()
            process_env.update(self.env)
            if self.spdk_base_lba is not None:
                process_env["SPDK_BASE_LBA"] = str(self.spdk_base_lba)
            try:
                completed = subprocess.run(
                    command, env=process_env, text=True, capture_output=True,
                    check=False, timeout=timeout,
                )
            except subprocess.TimeoutExpired as error:
                raise QuiverError(f"quiver_search exceeded the {timeout:g} second timeout") from error
            if completed.returncode != 0:
                detail = completed.stderr.strip() or completed.stdout.strip()
                raise QuiverError(f"quiver_search exited with code {completed.returncode}: {detail}")

            ids = self._read_bin(result_prefix.with_name("result_ids.bin"), np.int32)
            distances = self._read_bin(result_prefix.with_name("result_distances.bin"), np.float32)
            expected = (array.shape[0], topk)
            if ids.shape != expected or distances.shape != expected:
                raise QuiverError(
                    f"unexpected result shape: ids={ids.shape}, "
                    f"distances={distances.shape}, expected={expected}"
                )
            return ids, distances

    def _materialize_ssd_list(self, work: Path) -> Path | None:
        if self.ssd_list_file:
            return self.ssd_list_file
        if not self.ssds:
            return None
        path = work / "ssds.txt"
        path.write_text("".join(f"{ssd}\n" for ssd in self.ssds), encoding="ascii")
        return path

    @staticmethod
    def _write_bin(path: Path, values: npt.NDArray[np.generic]) -> None:
        with path.open("wb") as output:
            output.write(struct.pack("<ii", values.shape[0], values.shape[1]))
            output.write(values.tobytes(order="C"))

    @staticmethod
    def _read_bin(path: Path, dtype: npt.DTypeLike) -> npt.NDArray[np.generic]:
        if not path.is_file():
            raise QuiverError(f"quiver_search did not create {path.name}")
        with path.open("rb") as source:
            header = source.read(8)
            if len(header) != 8:
                raise QuiverError(f"invalid result header in {path}")
            count, dims = struct.unpack("<ii", header)
            if count < 0 or dims < 0:
                raise QuiverError(f"invalid result dimensions in {path}")
            values = np.fromfile(source, dtype=np.dtype(dtype).newbyteorder("<"))
        if values.size != count * dims:
            raise QuiverError(f"truncated result data in {path}")
        return values.reshape(count, dims)

    @staticmethod
    def _positive(value: int, name: str) -> int:
        value = int(value)
        if value <= 0:
            raise ValueError(f"{name} must be positive")
        return value

    @staticmethod
    def _find_binary(binary: str | os.PathLike[str] | None) -> Path | None:
        """External engine path, or None for the in-process C-ABI engine."""
        candidates: list[Path] = []
        if binary:
            candidates.append(Path(binary).expanduser())
        elif os.environ.get("QUIVER_BINARY"):
            candidates.append(Path(os.environ["QUIVER_BINARY"]).expanduser())
        else:
            return None
        for candidate in candidates:
            resolved = candidate.resolve()
            if resolved.is_file() and os.access(resolved, os.X_OK):
                return resolved
        searched = ", ".join(str(path) for path in candidates) or "PATH"
        raise QuiverError(f"quiver_search executable not found (searched: {searched})")


# ---- helpers around the C ABI ---------------------------------------------

def build_index(
    base: npt.ArrayLike,
    out_prefix: str | os.PathLike[str],
    *,
    R: int = 64,
    L: int = 100,
    alpha: float = 1.2,
    num_chunks: int = 32,
    kmeans_iters: int = 15,
    pq_train_max: int = 262144,
    seed: int = 0x5EED5EED,
    threads: int = 0,
    passes: int = 2,
) -> None:
    """Build a DiskANN-format index (disk.index + PQ files) on the CPU."""
    arr = np.ascontiguousarray(base)
    if arr.ndim != 2:
        raise ValueError("base must be 2D")
    dtype = {np.dtype("u1"): _lib.QV_UINT8, np.dtype("i1"): _lib.QV_INT8,
             np.dtype("<f4"): _lib.QV_FLOAT}.get(arr.dtype)
    if dtype is None:
        raise ValueError("base dtype must be uint8, int8 or float32")
    p = _lib.default_build_params()
    p.R, p.L, p.alpha, p.num_chunks = R, L, alpha, num_chunks
    p.kmeans_iters, p.pq_train_max, p.seed, p.threads, p.passes = kmeans_iters, pq_train_max, seed, threads, passes
    _lib.check(_lib.load().qv_build_index_cpu(arr.ctypes.data, dtype, arr.shape[0], arr.shape[1],
                                              C.byref(p), str(out_prefix).encode()))


def build_nav(
    rows: npt.ArrayLike,
    ids: npt.ArrayLike,
    out_dir: str | os.PathLike[str],
    *,
    R: int = 28,
    L: int = 64,
    alpha: float = 1.2,
    seed: int = 0x5EED5EED,
    threads: int = 0,
    passes: int = 2,
) -> None:
    """Build a navigation graph over `rows` (a sample of the base vectors whose
    base ids are `ids`) and write nav_index, nav_index.data and map.txt."""
    arr = np.ascontiguousarray(rows)
    idv = np.ascontiguousarray(ids, dtype=np.int32)
    if arr.ndim != 2 or idv.shape != (arr.shape[0],):
        raise ValueError("rows must be 2D and ids one per row")
    dtype = {np.dtype("u1"): _lib.QV_UINT8, np.dtype("i1"): _lib.QV_INT8,
             np.dtype("<f4"): _lib.QV_FLOAT}.get(arr.dtype)
    if dtype is None:
        raise ValueError("rows dtype must be uint8, int8 or float32")
    if not 1 <= R <= 32:
        raise ValueError("R must be in [1, 32] (the nav graph's row limit)")
    p = _lib.default_build_params()
    p.R, p.L, p.alpha, p.seed, p.threads, p.passes = R, L, alpha, seed, threads, passes
    Path(out_dir).mkdir(parents=True, exist_ok=True)
    _lib.check(_lib.load().qv_build_nav(arr.ctypes.data, idv.ctypes.data, arr.shape[0], arr.shape[1], dtype,
                                        C.byref(p), str(out_dir).encode()))


def mixture(rows: int, dim: int, *, data_type: str = "uint8", num_centers: int = 1024,
            seed: int = 1, first_row: int = 0, center_lo: float = 32.0,
            center_hi: float = 224.0, sigma: float = 20.0,
            normalize: bool = True) -> npt.NDArray[np.generic]:
    """Rows of the seeded Gaussian-mixture generator (host side)."""
    m = _lib.Mixture(seed, num_centers, dim, _lib.QV_UINT8 if data_type == "uint8" else _lib.QV_FLOAT,
                     center_lo, center_hi, sigma, 1 if normalize else 0)
    out = np.empty((rows, dim), dtype=np.uint8 if data_type == "uint8" else np.float32)
    _lib.check(_lib.load().qv_mixture_fill_host(C.byref(m), first_row, rows, out.ctypes.data))
    return out
