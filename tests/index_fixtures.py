"""Hand-built DiskANN-format indexes for known-answer tests.

An independent Python writer of the layout the reference reads
(bin/common/metadata.hpp:15-72, src/shared/index/pq_search.cu:62-114,
node records per src/quiver/kernel_core/kernel_helpers.cuh:257-279).
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

PAGE = 4096


def write_index(path_prefix: Path, vectors: np.ndarray, adjacency: list[list[int]], medoid: int,
                R: int, pivots: np.ndarray, centroid: np.ndarray, chunk_offsets: np.ndarray,
                codes: np.ndarray) -> None:
    n, dim = vectors.shape
    data_size = vectors.dtype.itemsize * dim
    node_size = data_size + 4 + 4 * R
    npp = PAGE // node_size
    num_pages = (n + npp - 1) // npp
    out = bytearray(PAGE * (num_pages + 1))
    struct.pack_into("<II", out, 0, 9, 1)
    struct.pack_into("<9Q", out, 8, n, dim, medoid, node_size, npp, 0, 0, 0, len(out))
    for v in range(n):
        off = PAGE * (1 + v // npp) + (v % npp) * node_size
        out[off:off + data_size] = vectors[v].tobytes()
        nb = adjacency[v]
        assert len(nb) <= R
        struct.pack_into(f"<I{len(nb)}I", out, off + data_size, len(nb), *nb)
    Path(str(path_prefix) + "_disk.index").write_bytes(bytes(out))

    M = len(chunk_offsets) - 1
    pv = np.ascontiguousarray(pivots, np.float32)
    ce = np.ascontiguousarray(centroid, np.float32)
    co = np.ascontiguousarray(chunk_offsets, np.int32)
    o0 = 4096
    o1 = o0 + 8 + pv.nbytes
    o2 = o1 + 8 + ce.nbytes
    o3 = o2 + 8 + co.nbytes
    meta = bytearray(4096)
    struct.pack_into("<ii4Q", meta, 0, 4, 1, o0, o1, o2, o3)
    body = (struct.pack("<ii", 256, dim) + pv.tobytes() + struct.pack("<ii", dim, 1) + ce.tobytes()
            + struct.pack("<ii", M + 1, 1) + co.tobytes())
    Path(str(path_prefix) + "_pq_pivots.bin").write_bytes(bytes(meta) + body)
    cd = np.ascontiguousarray(codes, np.uint8)
    Path(str(path_prefix) + "_pq_compressed.bin").write_bytes(struct.pack("<ii", n, M) + cd.tobytes())


def exact_pq(vectors: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """One-chunk-per-dimension PQ whose pivots are the values 0..255, so the
    ADC distance equals the exact squared L2 of uint8 data."""
    n, dim = vectors.shape
    pivots = np.tile(np.arange(256, dtype=np.float32)[:, None], (1, dim))
    centroid = np.zeros(dim, np.float32)
    offsets = np.arange(dim + 1, dtype=np.int32)
    codes = vectors.astype(np.uint8)
    return pivots, centroid, offsets, codes


def write_nav(nav_dir: Path, data: np.ndarray, graph: np.ndarray, mapping: np.ndarray, start: int) -> None:
    """The three nav-graph files NavGraph::init reads (src/shared/index/
    nav_graph.cu:12-71): nav_index.data (i32 num_node, i32 dims, vectors),
    map.txt (one base id per line), nav_index (u64 file size, u32 max degree,
    u32 start, u64 frozen points, then per node a u32 degree and its ids)."""
    d = Path(nav_dir)
    d.mkdir(parents=True, exist_ok=True)
    n, dims = data.shape
    (d / "nav_index.data").write_bytes(struct.pack("<ii", n, dims) + np.ascontiguousarray(data).tobytes())
    (d / "map.txt").write_text("".join(f"{int(x)}\n" for x in mapping))
    max_m = graph.shape[1]
    body = bytearray()
    for i in range(n):
        nb = [int(v) for v in graph[i] if v >= 0]
        body += struct.pack(f"<I{len(nb)}I", len(nb), *nb)
    (d / "nav_index").write_bytes(struct.pack("<QIIQ", 24 + len(body), max_m, start, 0) + bytes(body))
