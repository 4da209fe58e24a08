"""The run_persistent_search binding (quiver-ae_amd/compat/).

* quiver_hip_shim.cpp -- the function a reference maintainer builds in place
  of src/quiver/search.cu -- must compile against the reference's own headers
  (src/quiver/search.cuh and what it includes).  Those headers are CUDA
  sources: the one CUDA-toolkit macro they use, __align__ (which nvcc
  predefines), is given on the command line; nothing else is supplied.  CPU
  only, skipped where the reference checkout is absent (the GPU box).
* bin/run_persistent_search_test calls qv_compat::run_persistent_search with
  the reference's argument list (an index held in host memory, PQSearchData's
  tables, early-exit and per-step-recall options); its results must equal the
  oracle's (runs on the MI355X).
* qv_index_set_nav (a shared::NavGraph's host arrays) must search exactly like
  qv_index_load_nav of the same graph's files (runs on the MI355X).
"""
from __future__ import annotations

import ctypes as C
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import qv_oracle as O

ROOT = Path(__file__).resolve().parents[1]
REFERENCE = Path("/root/reference")
DRIVER = ROOT / "quiver-ae_amd" / "bin" / "run_persistent_search_test"


@pytest.mark.skipif(not (REFERENCE / "src" / "quiver" / "search.cuh").is_file(),
                    reason="reference checkout not present")
def test_shim_compiles_against_reference_headers():
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    r = subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-std=c++17", "-fsyntax-only",
                        "-D__align__(n)=__attribute__((aligned(n)))", f"-I{REFERENCE / 'src'}",
                        f"-I{ROOT / 'include'}", f"-I{ROOT / 'quiver-ae_amd' / 'compat'}",
                        str(ROOT / "quiver-ae_amd" / "compat" / "quiver_hip_shim.cpp")],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr


def _bin(path: Path, arr: np.ndarray) -> None:
    path.write_bytes(struct.pack("<ii", *arr.shape) + np.ascontiguousarray(arr).tobytes())


def _read(path: Path, dtype) -> np.ndarray:
    raw = path.read_bytes()
    n, d = struct.unpack("<ii", raw[:8])
    return np.frombuffer(raw[8:], dtype=dtype).reshape(n, d)


@pytest.mark.gpu
@pytest.mark.parametrize("policy", [0, 2])
def test_adapter_matches_oracle(small_u8_index, tmp_path, policy):
    ix = small_u8_index
    q = ix["queries"][:150]
    _bin(tmp_path / "q.u8bin", q)
    print(f"[gpu] run_persistent_search adapter policy={policy}", flush=True)
    r = subprocess.run([str(DRIVER), str(ix["dir"]), str(tmp_path / "q.u8bin"), "64", str(policy),
                        str(tmp_path / "out")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, ofound, _ = O.search(host, q.astype(np.float32), 10, 64,
                                       early_exit=O.EXIT_GPRUNING if policy == 2 else O.EXIT_NONE)
    np.testing.assert_array_equal(_read(tmp_path / "out_ids.bin", "<i4"), oids)
    np.testing.assert_array_equal(_read(tmp_path / "out_distances.bin", "<f4"), odists)
    np.testing.assert_array_equal(_read(tmp_path / "out_found.bin", "<i4")[:, 0], ofound)


@pytest.mark.gpu
def test_adapter_per_step_recall_matches_oracle(small_u8_index, tmp_path):
    ix = small_u8_index
    q = ix["queries"][:150]
    gt = np.ascontiguousarray(ix["gt"][:150], np.int32)
    _bin(tmp_path / "q.u8bin", q)
    _bin(tmp_path / "gt.ibin", gt)
    print("[gpu] run_persistent_search adapter per-step recall", flush=True)
    r = subprocess.run([str(DRIVER), str(ix["dir"]), str(tmp_path / "q.u8bin"), "96", "0", str(tmp_path / "out"),
                        str(tmp_path / "gt.ibin"), "0.7", str(tmp_path / "steps.csv")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, _, _, _, ostep, ohits = O.search(host, q.astype(np.float32), 10, 96, early_exit=O.EXIT_NONE,
                                           step_recall=(gt, O.required_hits(0.7, 10)))
    np.testing.assert_array_equal(_read(tmp_path / "out_ids.bin", "<i4"), oids)
    rows = [line.split(",") for line in (tmp_path / "steps.csv").read_text().splitlines()[1:]]
    np.testing.assert_array_equal([int(x[1]) for x in rows], ostep)
    np.testing.assert_array_equal([int(x[2]) for x in rows], ohits)
    assert "required_hits=7" in r.stdout


@pytest.mark.gpu
def test_set_nav_equals_load_nav(small_u8_index, tmp_path):
    import quiver
    from quiver import _lib

    L = _lib.load()
    ix = small_u8_index
    base = ix["base"]
    sample = np.arange(5, base.shape[0], 13, dtype=np.int32)
    quiver.build_nav(base[sample], sample, tmp_path / "nav", R=28, L=48, threads=0)
    nav = O.HostNav.from_dir(tmp_path / "nav", "uint8")
    q = np.ascontiguousarray(ix["queries"][:200], np.float32)
    out = []
    print("[gpu] qv_index_set_nav vs qv_index_load_nav", flush=True)
    for how in ("files", "arrays"):
        h = C.c_void_p()
        _lib.check(L.qv_index_open(str(ix["dir"]).encode(), b"uint8", b"heap", None, 0, C.byref(h)))
        try:
            if how == "files":
                _lib.check(L.qv_index_load_nav(h, str(tmp_path / "nav").encode()))
            else:
                _lib.check(L.qv_index_set_nav(h, nav.data.ctypes.data, nav.graph.ctypes.data,
                                              nav.mapping.ctypes.data, nav.num_node, nav.max_m, nav.start))
            ids = np.empty((200, 10), np.int32)
            dists = np.empty((200, 10), np.float32)
            hops = np.empty(200, np.int32)
            o = _lib.default_search_opts()
            o.early_exit = _lib.QV_EXIT_NONE
            _lib.check(L.qv_search(h, q.ctypes.data, 200, q.shape[1], 10, 64, C.byref(o), ids.ctypes.data,
                                   dists.ctypes.data, None, None))
            _lib.check(L.qv_last_hops(h, hops.ctypes.data, 200))
            out.append((ids, dists, hops))
            bad = nav.graph.copy()
            bad[0, 0] = nav.num_node  # an id past the graph is refused
            assert L.qv_index_set_nav(h, nav.data.ctypes.data, bad.ctypes.data, nav.mapping.ctypes.data,
                                      nav.num_node, nav.max_m, nav.start) == _lib.QV_EINDEX
        finally:
            L.qv_index_close(h)
    for a, b in zip(*out):
        np.testing.assert_array_equal(a, b)
    oids, _, _, _ = O.search(O.HostIndex.from_files(ix["dir"], "uint8"), q, 10, 64, early_exit=O.EXIT_NONE,
                             nav=nav)
    np.testing.assert_array_equal(out[1][0], oids)
