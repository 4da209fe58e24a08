"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module, always as the test oracle of the HIP path.  It reads DiskANN-format
index files with its own NumPy reader (independent of the library's C++
reader) and calls the C restatement in qv_oracle.c.
"""
from __future__ import annotations

import ctypes as C
import struct
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "build" / "libqv_oracle.so"
REF_RECALL = HERE / "_ref" / "librecall_ref.so"

UINT8, FLOAT, INT8 = 0, 1, 2
EXIT_NONE, EXIT_GPRUNING = 0, 2
PAGE = 4096


class OracleIndex(C.Structure):
    _fields_ = [
        ("dtype", C.c_int),
        ("dim", C.c_int),
        ("num_points", C.c_int64),
        ("max_m", C.c_int),
        ("medoid", C.c_int64),
        ("node_size", C.c_int64),
        ("nodes_per_page", C.c_int64),
        ("data_size", C.c_int64),
        ("pages", C.c_void_p),
        ("num_chunks", C.c_int),
        ("codes", C.c_void_p),
        ("centroid", C.c_void_p),
        ("pivots_t", C.c_void_p),
        ("chunk_id", C.c_void_p),
    ]


class SearchParams(C.Structure):
    _fields_ = [
        ("topk", C.c_int),
        ("ef_search", C.c_int),
        ("pipe_width", C.c_int),
        ("early_exit", C.c_int),
        ("gpruning_warmup", C.c_int),
        ("gpruning_patience", C.c_int),
        ("nav", C.c_void_p),
        ("sr_gt", C.c_void_p),
        ("sr_width", C.c_int),
        ("sr_count", C.c_int),
        ("sr_required", C.c_int),
        ("sr_step", C.c_void_p),
        ("sr_hits", C.c_void_p),
    ]


class OracleNav(C.Structure):
    _fields_ = [
        ("dtype", C.c_int),
        ("dim", C.c_int),
        ("num_node", C.c_int64),
        ("max_m", C.c_int),
        ("start", C.c_int),
        ("data", C.c_void_p),
        ("graph", C.c_void_p),
        ("mapping", C.c_void_p),
    ]


_lib = None


def load() -> C.CDLL:
    """Load the oracle library, building it with make when it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.is_file():
        subprocess.run(["make", "-C", str(HERE), "-s"], check=True)
    lib = C.CDLL(str(LIB))
    P = C.c_void_p
    lib.qvo_lut_build_raw.argtypes = [C.c_int, C.c_int, P, P, P, P, P, P]
    lib.qvo_lut_build_raw.restype = None
    lib.qvo_adc.argtypes = [P, C.c_int, P]
    lib.qvo_adc.restype = C.c_float
    lib.qvo_exact_l2.argtypes = [P, P, C.c_int, C.c_int]
    lib.qvo_exact_l2.restype = C.c_float
    lib.qvo_search_one.argtypes = [C.POINTER(OracleIndex), P, C.POINTER(SearchParams), P, P, P, P]
    lib.qvo_search_one.restype = C.c_int
    lib.qvo_search_trace.argtypes = [C.POINTER(OracleIndex), P, C.POINTER(SearchParams), P, P, P, P, P, C.c_int]
    lib.qvo_search_trace.restype = C.c_int
    lib.qvo_search.argtypes = [C.POINTER(OracleIndex), P, C.c_int64, C.POINTER(SearchParams), C.c_int,
                               P, P, P, P]
    lib.qvo_search.restype = C.c_int
    lib.qvo_search_timed.argtypes = [C.POINTER(OracleIndex), P, C.c_int64, C.POINTER(SearchParams), C.c_int,
                                     P, P, P, P, P]
    lib.qvo_search_timed.restype = C.c_int
    lib.qvo_recall.argtypes = [P, P, C.c_int64, C.c_int, C.c_int]
    lib.qvo_recall.restype = C.c_double
    lib.qvo_adc_topk.argtypes = [P, C.c_int, P, P, C.c_int64, C.c_int, P, P, C.POINTER(C.c_double)]
    lib.qvo_adc_topk.restype = None
    lib.qvo_ground_truth.argtypes = [P, C.c_int, C.c_int64, C.c_int, P, C.c_int64, C.c_int, C.c_int, P, P]
    lib.qvo_ground_truth.restype = None
    lib.qvo_nav_entry.argtypes = [C.POINTER(OracleNav), P, C.c_int64]
    lib.qvo_nav_entry.restype = C.c_int64
    _lib = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _read_bin_section(path: Path, offset: int, dtype) -> np.ndarray:
    with path.open("rb") as f:
        f.seek(offset)
        nr, nc = struct.unpack("<ii", f.read(8))
        data = np.frombuffer(f.read(nr * nc * np.dtype(dtype).itemsize), dtype=dtype)
    return data.reshape(nr, nc)


@dataclass
class HostIndex:
    """A DiskANN-format index held in host memory for the oracle."""

    dtype: int
    dim: int
    n: int
    R: int
    medoid: int
    node_size: int
    npp: int
    data_size: int
    pages: np.ndarray        # uint8 [num_pages * 4096], header page excluded
    codes: np.ndarray        # uint8 [n, M]
    centroid: np.ndarray     # float32 [d]
    pivots: np.ndarray       # float32 [256, d]
    pivots_t: np.ndarray     # float32 [d, 256]
    chunk_offsets: np.ndarray
    chunk_id: np.ndarray     # int32 [d]

    @property
    def M(self) -> int:
        return int(self.codes.shape[1])

    @classmethod
    def from_files(cls, index_dir: str | Path, data_type: str) -> "HostIndex":
        d = Path(index_dir)
        idx = sorted(d.glob("*_disk.index")) or [d / "disk.index"]
        piv = sorted(d.glob("*_pq_pivots.bin")) or [d / "pq_pivots.bin"]
        index_file, pivots_file = idx[0], piv[0]
        prefix = str(pivots_file)[: -len("_pivots.bin")]
        dt = {"uint8": UINT8, "float": FLOAT, "float32": FLOAT, "int8": INT8}[data_type]
        esz = 4 if dt == FLOAT else 1
        raw = np.fromfile(index_file, dtype=np.uint8)
        meta = np.frombuffer(raw[8:8 + 64].tobytes(), dtype="<u8")
        n, dim, medoid, node_len, npp = (int(x) for x in meta[:5])
        R = (node_len - dim * esz) // 4 - 1
        num_pages = (n + npp - 1) // npp
        pages = np.ascontiguousarray(raw[PAGE:PAGE * (num_pages + 1)])
        codes = np.ascontiguousarray(_read_bin_section(Path(prefix + "_compressed.bin"), 0, np.uint8))
        offs = _read_bin_section(pivots_file, 0, "<u8").ravel()
        ci = 3 if len(offs) == 5 else 2
        pivots = np.ascontiguousarray(_read_bin_section(pivots_file, int(offs[0]), "<f4"))
        centroid = np.ascontiguousarray(_read_bin_section(pivots_file, int(offs[1]), "<f4").ravel())
        co = _read_bin_section(pivots_file, int(offs[ci]), "<i4").ravel()
        chunk_id = np.full(dim, -1, dtype=np.int32)
        for i in range(len(co) - 1):
            chunk_id[co[i]:co[i + 1]] = i
        return cls(dt, dim, n, R, medoid, node_len, npp, dim * esz, pages, codes, centroid,
                   pivots, np.ascontiguousarray(pivots.T), co.astype(np.int32), chunk_id)

    @classmethod
    def from_arrays(cls, dtype: int, dim: int, n: int, R: int, medoid: int, pages: np.ndarray,
                    codes: np.ndarray, centroid: np.ndarray, pivots: np.ndarray,
                    chunk_offsets: np.ndarray) -> "HostIndex":
        """An index already in host memory (page image without the header page)."""
        esz = 4 if dtype == FLOAT else 1
        node_size = dim * esz + 4 + 4 * R
        npp = PAGE // node_size
        co = np.ascontiguousarray(chunk_offsets, np.int32)
        chunk_id = np.full(dim, -1, dtype=np.int32)
        for i in range(len(co) - 1):
            chunk_id[co[i]:co[i + 1]] = i
        piv = np.ascontiguousarray(pivots, np.float32)
        return cls(dtype, dim, n, R, medoid, node_size, npp, dim * esz, np.ascontiguousarray(pages),
                   np.ascontiguousarray(codes), np.ascontiguousarray(centroid, np.float32), piv,
                   np.ascontiguousarray(piv.T), co, chunk_id)

    def node_record(self, v: int) -> np.ndarray:
        off = (v // self.npp) * PAGE + (v % self.npp) * self.node_size
        return self.pages[off:off + self.node_size]

    def vector(self, v: int) -> np.ndarray:
        rec = self.node_record(v)[: self.data_size]
        return rec.view({UINT8: np.uint8, INT8: np.int8, FLOAT: np.float32}[self.dtype])

    def neighbors(self, v: int) -> np.ndarray:
        rec = self.node_record(v)[self.data_size:].view(np.uint32)
        return rec[1:1 + int(rec[0])]

    def base(self) -> np.ndarray:
        return np.stack([self.vector(v) for v in range(self.n)])

    def c_struct(self) -> OracleIndex:
        return OracleIndex(self.dtype, self.dim, self.n, self.R, self.medoid, self.node_size, self.npp,
                           self.data_size, _ptr(self.pages), self.M, _ptr(self.codes),
                           _ptr(self.centroid), _ptr(self.pivots_t), _ptr(self.chunk_id))


@dataclass
class HostNav:
    """A navigation graph (nav_index, nav_index.data, map.txt) in host memory."""

    dtype: int
    dim: int
    num_node: int
    max_m: int
    start: int
    data: np.ndarray      # [num_node, dim] of the base element type
    graph: np.ndarray     # int32 [num_node, max_m], -1 after each degree
    mapping: np.ndarray   # int32 [num_node]

    @classmethod
    def from_dir(cls, nav_dir: str | Path, data_type: str) -> "HostNav":
        """Reads the three files the reference's NavGraph::init reads
        (src/shared/index/nav_graph.cu:12-71)."""
        d = Path(nav_dir)
        dt = {"uint8": UINT8, "float": FLOAT, "float32": FLOAT, "int8": INT8}[data_type]
        np_dt = {UINT8: np.uint8, INT8: np.int8, FLOAT: np.float32}[dt]
        raw = np.fromfile(d / "nav_index.data", dtype=np.uint8)
        num_node, dim = (int(x) for x in np.frombuffer(raw[:8].tobytes(), dtype="<i4"))
        data = np.frombuffer(raw[8:].tobytes(), dtype=np_dt)[: num_node * dim].reshape(num_node, dim)
        mapping = np.array([int(x) for x in (d / "map.txt").read_text().split()[:num_node]], np.int32)
        g = np.fromfile(d / "nav_index", dtype="<u4")
        max_m, start = int(g[2]), int(g[3])
        graph = np.full((num_node, max_m), -1, np.int32)
        pos = 6
        for i in range(num_node):
            deg = int(g[pos])
            graph[i, :deg] = g[pos + 1:pos + 1 + deg].astype(np.int32)
            pos += 1 + deg
        return cls(dt, dim, num_node, max_m, start, np.ascontiguousarray(data), graph, mapping)

    @classmethod
    def from_arrays(cls, data: np.ndarray, graph: np.ndarray, mapping: np.ndarray,
                    start: int = 0) -> "HostNav":
        dt = {np.dtype("u1"): UINT8, np.dtype("i1"): INT8, np.dtype("<f4"): FLOAT}[data.dtype]
        g = np.ascontiguousarray(graph, np.int32)
        return cls(dt, int(data.shape[1]), int(data.shape[0]), int(g.shape[1]), int(start),
                   np.ascontiguousarray(data), g, np.ascontiguousarray(mapping, np.int32))

    def c_struct(self) -> OracleNav:
        return OracleNav(self.dtype, self.dim, self.num_node, self.max_m, self.start, _ptr(self.data),
                         _ptr(self.graph), _ptr(self.mapping))


def nav_entry(nav: HostNav, q: np.ndarray, fallback: int = -1) -> int:
    """Entry node (base id) that the nav search picks for the raw query q."""
    cs = nav.c_struct()
    qq = np.ascontiguousarray(q, np.float32)
    return int(load().qvo_nav_entry(C.byref(cs), _ptr(qq), fallback))


def required_hits(threshold: float, topk: int) -> int:
    """Hits a query needs to stop under per-step recall (search.cu:100-102)."""
    import math
    return max(1, min(topk, int(math.ceil(np.float32(threshold) * np.float32(topk) - np.float32(1e-6)))))


def search(ix: HostIndex, queries: np.ndarray, topk: int, ef: int, *, pipe_width: int = 1,
           early_exit: int = EXIT_GPRUNING, warmup: int = 10, patience: int = 8, threads: int = 0,
           nav: HostNav | None = None, seconds: np.ndarray | None = None,
           step_recall: tuple[np.ndarray, int] | None = None):
    """Oracle search: returns (ids int32 [n,k], dists float32 [n,k], found, hops).
    With `nav`, each query starts from its nav-graph entry instead of the medoid.
    With `seconds` (float64 [n]), each query's wall time is written there.
    With `step_recall` = (ground truth int32 [count, width], required hits),
    each query stops once that many of its top-k ids are in its ground-truth
    row, and (step, hits) arrays are returned after the four above."""
    lib = load()
    q = np.ascontiguousarray(queries, dtype=np.float32)
    n = q.shape[0]
    ids = np.empty((n, topk), np.int32)
    dists = np.empty((n, topk), np.float32)
    found = np.empty(n, np.int32)
    hops = np.empty(n, np.int32)
    ns = nav.c_struct() if nav is not None else None
    p = SearchParams(topk, ef, pipe_width, early_exit, warmup, patience,
                     C.cast(C.pointer(ns), C.c_void_p) if ns is not None else None)
    if step_recall is not None:
        sr_gt = np.ascontiguousarray(step_recall[0], np.int32)
        sr_step = np.empty(n, np.int32)
        sr_hits = np.empty(n, np.int32)
        p.sr_gt, p.sr_width, p.sr_count = sr_gt.ctypes.data, sr_gt.shape[1], sr_gt.shape[0]
        p.sr_required = int(step_recall[1])
        p.sr_step, p.sr_hits = sr_step.ctypes.data, sr_hits.ctypes.data
    cs = ix.c_struct()
    if seconds is not None:
        if seconds.dtype != np.float64 or seconds.shape != (n,) or not seconds.flags.c_contiguous:
            raise ValueError("seconds must be a contiguous float64 array of one entry per query")
        rc = lib.qvo_search_timed(C.byref(cs), _ptr(q), n, C.byref(p), threads, _ptr(ids), _ptr(dists),
                                  _ptr(found), _ptr(hops), _ptr(seconds))
    else:
        rc = lib.qvo_search(C.byref(cs), _ptr(q), n, C.byref(p), threads, _ptr(ids), _ptr(dists),
                            _ptr(found), _ptr(hops))
    if rc != 0:
        raise RuntimeError(f"oracle search failed with status {rc}")
    if step_recall is not None:
        return ids, dists, found, hops, sr_step, sr_hits
    return ids, dists, found, hops


def search_trace(ix: HostIndex, query: np.ndarray, topk: int, ef: int, *, pipe_width: int = 1,
                 early_exit: int = EXIT_NONE, warmup: int = 10, patience: int = 8, cap: int = 4096,
                 step_recall: tuple[np.ndarray, int] | None = None):
    """One query; returns (ids, dists, found, hops, expanded) where expanded[s]
    is the node expanded at step s + 1 (the entry first).  With `step_recall`
    = (ground-truth row int32 [width], required hits), (step, hits) follow."""
    lib = load()
    q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
    ids = np.empty(topk, np.int32)
    dists = np.empty(topk, np.float32)
    found = np.empty(1, np.int32)
    hops = np.empty(1, np.int32)
    trace = np.full(cap, -1, np.int32)
    p = SearchParams(topk, ef, pipe_width, early_exit, warmup, patience, None)
    if step_recall is not None:
        sr_gt = np.ascontiguousarray(step_recall[0], np.int32).reshape(1, -1)
        sr_out = np.full(2, -7, np.int32)
        p.sr_gt, p.sr_width, p.sr_count = sr_gt.ctypes.data, sr_gt.shape[1], 1
        p.sr_required = int(step_recall[1])
        p.sr_step, p.sr_hits = sr_out.ctypes.data, sr_out.ctypes.data + 4
    cs = ix.c_struct()
    rc = lib.qvo_search_trace(C.byref(cs), _ptr(q), C.byref(p), _ptr(ids), _ptr(dists), _ptr(found),
                              _ptr(hops), _ptr(trace), cap)
    if rc != 0:
        raise RuntimeError(f"oracle search failed with status {rc}")
    h = int(hops[0])
    out = (ids, dists, int(found[0]), h, [int(v) for v in trace[:min(h, cap)]])
    if step_recall is not None:
        return out + (int(sr_out[0]), int(sr_out[1]))
    return out


def lut(dim: int, centroid: np.ndarray, pivots_t: np.ndarray, chunk_id: np.ndarray,
        q: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    lib = load()
    M = int(chunk_id.max()) + 1
    out = np.empty((M, 256), np.float32)
    qu = np.empty(dim, np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    lib.qvo_lut_build_raw(dim, M, _ptr(np.ascontiguousarray(centroid, np.float32)),
                          _ptr(np.ascontiguousarray(pivots_t, np.float32)),
                          _ptr(np.ascontiguousarray(chunk_id, np.int32)), _ptr(q), _ptr(out), _ptr(qu))
    return out, qu


def adc(lut_tbl: np.ndarray, code_row: np.ndarray) -> float:
    t = np.ascontiguousarray(lut_tbl, np.float32)
    c = np.ascontiguousarray(code_row, np.uint8)
    return float(load().qvo_adc(_ptr(t), c.shape[0], _ptr(c)))


def exact_l2(q: np.ndarray, x: np.ndarray) -> float:
    dt = {np.dtype("u1"): UINT8, np.dtype("i1"): INT8, np.dtype("<f4"): FLOAT}[x.dtype]
    q = np.ascontiguousarray(q, np.float32)
    x = np.ascontiguousarray(x)
    return float(load().qvo_exact_l2(_ptr(q), _ptr(x), dt, q.shape[0]))


def recall(results: np.ndarray, gt: np.ndarray, k: int) -> float:
    r = np.ascontiguousarray(results, np.int32)
    g = np.ascontiguousarray(gt, np.int32)
    return float(load().qvo_recall(_ptr(r), _ptr(g), r.shape[0], g.shape[1], k))


def adc_topk(lut_tbl: np.ndarray, codes: np.ndarray, ids: np.ndarray, k: int):
    t = np.ascontiguousarray(lut_tbl, np.float32)
    c = np.ascontiguousarray(codes, np.uint8)
    i = np.ascontiguousarray(ids, np.int32)
    out_i = np.empty(k, np.int32)
    out_d = np.empty(k, np.float32)
    s = C.c_double(0.0)
    load().qvo_adc_topk(_ptr(t), c.shape[1], _ptr(c), _ptr(i), i.shape[0], k, _ptr(out_i), _ptr(out_d),
                        C.byref(s))
    return out_i, out_d, s.value


def ground_truth(base: np.ndarray, queries: np.ndarray, k: int, threads: int = 0):
    dt = {np.dtype("u1"): UINT8, np.dtype("i1"): INT8, np.dtype("<f4"): FLOAT}[base.dtype]
    b = np.ascontiguousarray(base)
    q = np.ascontiguousarray(queries, np.float32)
    ids = np.empty((q.shape[0], k), np.int32)
    dists = np.empty((q.shape[0], k), np.float32)
    load().qvo_ground_truth(_ptr(b), dt, b.shape[0], b.shape[1], _ptr(q), q.shape[0], k, threads,
                            _ptr(ids), _ptr(dists))
    return ids, dists


def reference_recall_lib():
    """The reference's own recall header compiled into oracle/_ref, or None."""
    if not REF_RECALL.is_file():
        return None
    lib = C.CDLL(str(REF_RECALL))
    lib.ref_calc_recall.argtypes = [C.c_void_p, C.c_void_p, C.c_long, C.c_long, C.c_int]
    lib.ref_calc_recall.restype = C.c_double
    lib.ref_query_hits.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.ref_query_hits.restype = C.c_int
    return lib
