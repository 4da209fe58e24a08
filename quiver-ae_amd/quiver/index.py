"""NumPy front end with the reference binding's interface
(python/quiver/index.py:27-264): ``IndexQuiver(index_dir, ...).search(queries,
topk, ef_search=...)`` returns ``(ids int32[n, topk], distances float32[n,
topk])``.

Two engines sit behind the one facade:

* ``_LibraryEngine`` (default): libquiver_hip's C ABI in this process; the
  graph, vectors and PQ codes stay resident in GPU memory between searches.
* ``_ProcessEngine`` (when ``binary=`` or ``QUIVER_BINARY`` names an
  executable): runs that ``quiver_search`` once per call with the reference's
  command-line contract -- query file in, ``<prefix>_ids.bin`` /
  ``<prefix>_distances.bin`` out -- so any engine speaking it can be plugged in.

Argument names, defaults, accepted values and error messages are the
reference binding's, because callers depend on them.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import tempfile
from dataclasses import dataclass
from pathlib import Path
from typing import Mapping, Sequence

import numpy as np
import numpy.typing as npt

from . import _lib
from ._binfile import read_matrix, write_matrix
from ._lib import QuiverError

# Element type of an index, by its canonical --data-type name: the dtype queries
# are converted to and the query-file suffix (python/quiver/index.py:18-23).
_ELEMENTS = {"float": ("<f4", ".fbin"), "uint8": ("u1", ".u8bin"), "int8": ("i1", ".i8bin")}
_TYPE_ALIASES = {"float32": "float"}
_POLICIES = ("gpruning", "none")
# The reference's --num-blocks default (python/quiver/index.py:45).
_REFERENCE_NUM_BLOCKS = 756


def _positive(name: str, value) -> int:
    number = int(value)
    if number <= 0:
        raise ValueError(f"{name} must be positive")
    return number


def _count_ssds(list_file: Path) -> int:
    """Lines naming an SSD: non-blank and not a '#' comment."""
    entries = (line.strip() for line in list_file.read_text().splitlines())
    return sum(1 for entry in entries if entry and entry[0] != "#")


@dataclass(frozen=True)
class _EngineKnobs:
    """The per-index engine settings both engines forward."""

    num_blocks: int
    queries_per_block: int
    pipe_width: int
    poll_threads: int
    runners_per_ssd: int


class _LibraryEngine:
    """Searches through libquiver_hip's C ABI on one GPU."""

    def __init__(self, owner: "IndexQuiver", device: int, graph_placement: str, search_kernel: str,
                 neighbour_codes: bool) -> None:
        self._owner = owner
        self._device = device
        self._placement = _lib.QV_GRAPH_HOST if graph_placement == "host" else _lib.QV_GRAPH_HBM
        self._kernel = _lib.KERNEL_NAMES[search_kernel]
        self._neighbour_codes = neighbour_codes
        self._handle: C.c_void_p | None = None
        _lib.load()  # a missing library fails here, not at the first search

    def handle(self) -> C.c_void_p:
        if self._handle is None:
            o = self._owner
            handle = C.c_void_p()
            _lib.check(_lib.load().qv_index_open_ex(
                str(o.index_dir).encode(), o.data_type.encode(), o.memory_backend.encode(), None,
                self._device, self._placement, C.byref(handle)))
            if self._neighbour_codes:
                try:
                    _lib.check(_lib.load().qv_index_neighbour_codes(handle, 1))
                except QuiverError:
                    _lib.load().qv_index_close(handle)
                    raise
            self._handle = handle
        return self._handle

    def _options(self, policy: str, timeout: float | None, skip_nav: bool) -> _lib.SearchOpts:
        knobs = self._owner._knobs
        opts = _lib.default_search_opts()
        opts.num_blocks = knobs.num_blocks
        opts.queries_per_block = knobs.queries_per_block
        opts.pipe_width = knobs.pipe_width
        opts.early_exit = _lib.QV_EXIT_GPRUNING if policy == "gpruning" else _lib.QV_EXIT_NONE
        opts.timeout_s = 0.0 if timeout is None else float(timeout)
        opts.skip_nav = int(skip_nav)
        opts.kernel = self._kernel
        # the admission knobs the reference engine reads from its environment
        # (src/quiver/search.cu:827-860)
        env = {**os.environ, **self._owner.env}
        if env.get("QUIVER_PREFEED"):
            opts.prefeed = int(env["QUIVER_PREFEED"])
        if env.get("QUIVER_ADMIT_MIN_BATCH"):
            opts.admit_min_batch = max(1, int(env["QUIVER_ADMIT_MIN_BATCH"]))
        return opts

    def search(self, queries: np.ndarray, topk: int, ef_search: int, policy: str,
               timeout: float | None, extra_args: Sequence[str]):
        extra = [str(a) for a in extra_args]
        skip_nav = "--skip-nav" in extra
        if any(a != "--skip-nav" for a in extra):
            raise QuiverError("extra_args other than --skip-nav need an external quiver_search binary")
        if self._owner.num_ssds:
            raise QuiverError("This binary was built without SPDK support")
        handle = self.handle()
        q = np.ascontiguousarray(queries, dtype=np.float32)  # load_queries_as_float
        n, dim = q.shape
        ids = np.empty((n, topk), np.int32)
        dists = np.empty((n, topk), np.float32)
        found = np.empty(n, np.int32)
        report = _lib.SearchReport()
        opts = self._options(policy, timeout, skip_nav)
        rc = _lib.load().qv_search(handle, q.ctypes.data, n, dim, topk, ef_search, C.byref(opts),
                                   ids.ctypes.data, dists.ctypes.data, found.ctypes.data, C.byref(report))
        if rc == _lib.QV_ETIMEDOUT and timeout is not None:
            raise QuiverError(f"quiver_search exceeded the {timeout:g} second timeout")
        _lib.check(rc)  # any other failure (the kernel's own watchdog included) with the library's text
        self._owner.last_report = report.as_dict()
        return ids, dists

    def close(self) -> None:
        if self._handle is not None:
            _lib.load().qv_index_close(self._handle)
            self._handle = None


class _ProcessEngine:
    """Runs an external quiver_search per call (bin/quiver_search.cu:58-320)."""

    def __init__(self, owner: "IndexQuiver", executable: Path) -> None:
        self._owner = owner
        self.executable = executable

    def _argv(self, query_file: Path, result_prefix: Path, topk: int, ef_search: int, policy: str,
              ssd_list: Path | None, extra_args: Sequence[str]) -> list[str]:
        o, k = self._owner, self._owner._knobs
        pairs = {
            "--index-dir": o.index_dir, "--data-type": o.data_type, "--memory-backend": o.memory_backend,
            "--query": query_file, "--result-prefix": result_prefix,
            "--topk": topk, "--ef-search": ef_search, "--early-exit-policy": policy,
            "--repeat": 1,  # one timed pass per call
            "--num-blocks": k.num_blocks, "--queries-per-block": k.queries_per_block,
            "--pipe-width": k.pipe_width, "--poll-threads": k.poll_threads,
            "--runners-per-ssd": k.runners_per_ssd,
        }
        if ssd_list is not None:
            pairs["--ssd-list-file"] = ssd_list
        argv = [str(self.executable)]
        for flag, value in pairs.items():
            argv += [flag, str(value)]
        return argv + [str(a) for a in extra_args]

    def _environment(self) -> dict[str, str]:
        env = dict(os.environ)
        env.update(self._owner.env)
        if self._owner.spdk_base_lba is not None:
            env["SPDK_BASE_LBA"] = str(self._owner.spdk_base_lba)
        return env

    def search(self, queries: np.ndarray, topk: int, ef_search: int, policy: str,
               timeout: float | None, extra_args: Sequence[str]):
        o = self._owner
        with tempfile.TemporaryDirectory(prefix="quiver-python-") as scratch:
            work = Path(scratch)
            query_file = work / ("queries" + o._query_suffix)
            write_matrix(query_file, queries)
            ssd_list = o.ssd_list_file
            if ssd_list is None and o.ssds:
                ssd_list = work / "ssds.txt"
                ssd_list.write_text("\n".join(o.ssds) + "\n", encoding="ascii")
            prefix = work / "result"
            argv = self._argv(query_file, prefix, topk, ef_search, policy, ssd_list, extra_args)
            with subprocess.Popen(argv, env=self._environment(), stdout=subprocess.PIPE,
                                  stderr=subprocess.PIPE, text=True) as proc:
                try:
                    out, err = proc.communicate(timeout=timeout)
                except subprocess.TimeoutExpired:
                    proc.kill()
                    proc.communicate()
                    raise QuiverError(f"quiver_search exceeded the {timeout:g} second timeout") from None
            if proc.returncode != 0:
                detail = err.strip() or out.strip()
                raise QuiverError(f"quiver_search exited with code {proc.returncode}: {detail}")
            ids = read_matrix(work / "result_ids.bin", "i4")
            dists = read_matrix(work / "result_distances.bin", "f4")
        want = (queries.shape[0], topk)
        if ids.shape != want or dists.shape != want:
            raise QuiverError(f"unexpected result shape: ids={ids.shape}, distances={dists.shape}, "
                              f"expected={want}")
        return ids, dists

    def close(self) -> None:
        pass


def _external_engine_path(binary: str | os.PathLike[str] | None) -> Path | None:
    """The external engine named by `binary` or QUIVER_BINARY; None selects
    the in-process engine.  A named path that is not an executable file is an
    error."""
    named = binary or os.environ.get("QUIVER_BINARY")
    if not named:
        return None
    path = Path(named).expanduser().resolve()
    if not (path.is_file() and os.access(path, os.X_OK)):
        raise QuiverError(f"quiver_search executable not found (searched: {Path(named).expanduser()})")
    return path


class IndexQuiver:
    """Search a Quiver index with NumPy arrays.

    The default engine keeps the graph, vectors and PQ codes resident in GPU
    memory (the heap memory backend, or the mmap one).  SSD options are
    accepted for compatibility; the SPDK backend is not part of this library,
    so searching with SSDs configured raises ``QuiverError`` unless an
    external ``binary`` is used.  Extra keyword arguments beyond the
    reference's: ``device``, ``graph_placement`` ("hbm" or "host"),
    ``search_kernel`` ("auto", "lut" or "shared-pivots") and
    ``neighbour_codes`` (store each node's neighbours' PQ code rows as one
    block in device memory, n * R * M bytes: the same results with fewer
    bytes read per hop; indexes with R <= 64 and M = 32 or 48).
    ``num_blocks`` left unset fills the GPU with concurrent query slots (an
    external ``binary`` gets the reference's 756); a number given is the slot
    count, as in the reference.  Results do not depend on it.
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
        num_blocks: int | None = None,
        queries_per_block: int = 1,
        pipe_width: int = 2,
        poll_threads: int = 6,
        runners_per_ssd: int = 1,
        env: Mapping[str, str] | None = None,
        device: int = 0,
        graph_placement: str = "hbm",
        search_kernel: str = "auto",
        neighbour_codes: bool = False,
    ) -> None:
        root = Path(index_dir).expanduser().resolve()
        if not root.is_dir():
            raise ValueError(f"index_dir is not a directory: {root}")
        self.index_dir = root

        canonical = _TYPE_ALIASES.get(data_type.lower(), data_type.lower())
        if canonical not in _ELEMENTS:
            raise ValueError("data_type must be float32, float, uint8, or int8")
        self.data_type = canonical
        dtype, self._query_suffix = _ELEMENTS[canonical]
        self._numpy_dtype = np.dtype(dtype)

        if ssds and ssd_list_file:
            raise ValueError("pass either ssds or ssd_list_file, not both")
        self.ssds = tuple(str(s).strip() for s in ssds or ())
        if "" in self.ssds:
            raise ValueError("SSD PCI addresses must not be empty")
        self.ssd_list_file = Path(ssd_list_file).expanduser().resolve() if ssd_list_file else None
        if self.ssd_list_file is not None and not self.ssd_list_file.is_file():
            raise ValueError(f"ssd_list_file does not exist: {self.ssd_list_file}")
        if spdk_base_lba is not None and spdk_base_lba < 0:
            raise ValueError("spdk_base_lba must be non-negative")
        self.spdk_base_lba = spdk_base_lba

        if memory_backend not in ("heap", "mmap"):
            raise ValueError("memory_backend must be heap or mmap")
        self.memory_backend = memory_backend
        if graph_placement not in ("hbm", "host"):
            raise ValueError("graph_placement must be hbm or host")
        self.graph_placement = graph_placement
        if search_kernel not in _lib.KERNEL_NAMES:
            raise ValueError("search_kernel must be auto, lut or shared-pivots")
        self.search_kernel = search_kernel
        self.neighbour_codes = bool(neighbour_codes)

        external = _external_engine_path(binary)
        # Unset, the library fills the GPU with query slots (0); an external
        # binary gets the reference's own default, 756.  The count changes
        # only how many queries run at once, never a query's results.
        if num_blocks is None:
            num_blocks = 0 if external is None else _REFERENCE_NUM_BLOCKS
        else:
            num_blocks = _positive("num_blocks", num_blocks)
        self._knobs = _EngineKnobs(
            num_blocks=num_blocks,
            queries_per_block=_positive("queries_per_block", queries_per_block),
            pipe_width=_positive("pipe_width", pipe_width),
            poll_threads=_positive("poll_threads", poll_threads),
            runners_per_ssd=_positive("runners_per_ssd", runners_per_ssd),
        )
        self.env = dict(env or {})
        self.device = int(device)
        self.last_report: dict | None = None
        self._engine = (_ProcessEngine(self, external) if external is not None
                        else _LibraryEngine(self, self.device, graph_placement, search_kernel,
                                       self.neighbour_codes))

    # the engine knobs, readable as attributes like the reference's
    num_blocks = property(lambda self: self._knobs.num_blocks)
    queries_per_block = property(lambda self: self._knobs.queries_per_block)
    pipe_width = property(lambda self: self._knobs.pipe_width)
    poll_threads = property(lambda self: self._knobs.poll_threads)
    runners_per_ssd = property(lambda self: self._knobs.runners_per_ssd)

    @property
    def binary(self) -> Path | None:
        """The external engine's path, or None for the in-process engine."""
        return self._engine.executable if isinstance(self._engine, _ProcessEngine) else None

    @property
    def num_ssds(self) -> int:
        if self.ssds:
            return len(self.ssds)
        return _count_ssds(self.ssd_list_file) if self.ssd_list_file else 0

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
        topk = _positive("topk", topk)
        ef_search = _positive("ef_search", ef_search)
        if early_exit_policy not in _POLICIES:
            raise ValueError("early_exit_policy must be gpruning or none")
        if timeout is not None and timeout <= 0:
            raise ValueError("timeout must be positive")
        batch = np.asarray(queries)
        if batch.ndim == 1:
            batch = batch[np.newaxis, :]
        if batch.ndim != 2 or 0 in batch.shape:
            raise ValueError("queries must be a non-empty 1D or 2D array")
        batch = np.ascontiguousarray(batch, dtype=self._numpy_dtype)
        return self._engine.search(batch, topk, ef_search, early_exit_policy, timeout, extra_args)

    # ---- in-process engine only -----------------------------------------
    def _library(self) -> _LibraryEngine:
        if not isinstance(self._engine, _LibraryEngine):
            raise QuiverError("this IndexQuiver runs an external quiver_search binary")
        return self._engine

    def info(self) -> dict:
        """Layout and placement of the opened index (qv_index_get_info)."""
        info = _lib.IndexInfo()
        _lib.check(_lib.load().qv_index_get_info(self._library().handle(), C.byref(info)))
        return {name: getattr(info, name) for name, _ in info._fields_}

    def load_nav(self, nav_dir: str | os.PathLike[str]) -> None:
        """Load (or replace) the navigation graph that picks each query's entry
        node (nav_index, nav_index.data, map.txt).  An index directory holding
        nav_index or nav/nav_index gets its graph at open without this call."""
        _lib.check(_lib.load().qv_index_load_nav(self._library().handle(), str(nav_dir).encode()))

    def close(self) -> None:
        engine = getattr(self, "_engine", None)
        if engine is not None:
            engine.close()

    def __enter__(self) -> "IndexQuiver":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


# ---- index construction and synthetic data (C ABI) ------------------------

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
