"""ctypes view of libquiver_hip.so (include/quiver_hip.h).

The library is loaded from ``quiver-ae_amd/lib`` (or ``QUIVER_HIP_LIB``).  A
missing library raises ``QuiverError``; nothing here falls back to Python.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path


class QuiverError(RuntimeError):
    """Raised when Quiver cannot execute or return valid search results."""


QV_OK = 0
QV_EINVAL = -1
QV_EIO = -2
QV_EHIP = -3
QV_ETIMEDOUT = -4
QV_EUNSUPPORTED = -5
QV_ENOMEM = -6
QV_EINDEX = -7

QV_UINT8 = 0
QV_FLOAT = 1
QV_INT8 = 2
QV_EXIT_NONE = 0
QV_EXIT_GPRUNING = 2
QV_ADMIT_STREAMING = 0
QV_ADMIT_BATCH = 1
QV_ADMIT_STATIC = 2
QV_GRAPH_HBM = 0
QV_GRAPH_HOST = 1
QV_STREAM_READ_BLOCKS = 4096
QV_NOALLOC_SCRATCH_BYTES = 12 * 1024 * 1024 + 256 + 16 * 1024
QV_NOALLOC_MAX_QUERIES = 1024 * 1024
QV_KERNEL_AUTO = 0
QV_KERNEL_LUT = 1
QV_KERNEL_SHARED_PIVOTS = 2
KERNEL_NAMES = {"auto": QV_KERNEL_AUTO, "lut": QV_KERNEL_LUT, "shared-pivots": QV_KERNEL_SHARED_PIVOTS}

PKG_ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = PKG_ROOT / "lib" / "libquiver_hip.so"
CLI_PATH = PKG_ROOT / "bin" / "quiver_search"


class IndexInfo(C.Structure):
    _fields_ = [
        ("num_data", C.c_int64),
        ("num_dims", C.c_int64),
        ("max_m0", C.c_int64),
        ("enter_point", C.c_int64),
        ("data_size", C.c_int64),
        ("node_size", C.c_int64),
        ("num_pages", C.c_int64),
        ("nodes_per_page", C.c_int64),
        ("data_type", C.c_int32),
        ("num_chunks", C.c_int32),
        ("device", C.c_int32),
        ("slots_per_cu", C.c_int32),
        ("device_bytes", C.c_int64),
        ("nav_nodes", C.c_int64),
        ("nav_max_m", C.c_int32),
        ("reserved", C.c_int32),
    ]


class SearchOpts(C.Structure):
    _fields_ = [
        ("num_blocks", C.c_int32),
        ("queries_per_block", C.c_int32),
        ("pipe_width", C.c_int32),
        ("early_exit", C.c_int32),
        ("gpruning_warmup", C.c_int32),
        ("gpruning_patience", C.c_int32),
        ("prefeed", C.c_int32),
        ("admit_min_batch", C.c_int32),
        ("admission", C.c_int32),
        ("device_buffers", C.c_int32),
        ("timeout_s", C.c_double),
        ("skip_nav", C.c_int32),
        ("kernel", C.c_int32),
        ("step_recall_gt", C.c_void_p),
        ("step_recall_gt_width", C.c_int32),
        ("step_recall_gt_count", C.c_int32),
        ("step_recall_threshold", C.c_float),
        ("step_recall_step", C.c_void_p),
        ("step_recall_hits", C.c_void_p),
        ("arrival_qps", C.c_double),
        ("arrival_batch", C.c_int32),
        ("reserved0", C.c_int32),
    ]


class SearchReport(C.Structure):
    _fields_ = [
        ("qps", C.c_double),
        ("search_time_s", C.c_double),
        ("lat_avg_ms", C.c_double),
        ("lat_p50_ms", C.c_double),
        ("lat_p90_ms", C.c_double),
        ("lat_p99_ms", C.c_double),
        ("lat_p999_ms", C.c_double),
        ("lat_max_ms", C.c_double),
        ("avg_hops", C.c_double),
        ("kernel_ms", C.c_double),
        ("num_blocks", C.c_int32),
        ("max_inflight", C.c_int32),
        ("early_stopped", C.c_int32),
        ("kernel", C.c_int32),
        ("total_hops", C.c_double),
        ("total_evals", C.c_double),
        ("tail_queries", C.c_int32),
        ("reserved1", C.c_int32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class BuildParams(C.Structure):
    _fields_ = [
        ("R", C.c_int32),
        ("L", C.c_int32),
        ("alpha", C.c_float),
        ("num_chunks", C.c_int32),
        ("kmeans_iters", C.c_int32),
        ("pq_train_max", C.c_int32),
        ("seed", C.c_uint64),
        ("threads", C.c_int32),
        ("passes", C.c_int32),
    ]


class Mixture(C.Structure):
    _fields_ = [
        ("seed", C.c_uint64),
        ("num_centers", C.c_int32),
        ("dim", C.c_int32),
        ("data_type", C.c_int32),
        ("center_lo", C.c_float),
        ("center_hi", C.c_float),
        ("sigma", C.c_float),
        ("normalize", C.c_int32),
    ]


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64

# name -> (restype, argtypes); every symbol declared in include/quiver_hip.h.
SIGNATURES = {
    "qv_index_open": (_I32, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int, C.POINTER(_P)]),
    "qv_index_open_ex": (_I32, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int, _I32, C.POINTER(_P)]),
    "qv_index_place_graph": (_I32, [_P, _I32]),
    "qv_index_from_memory": (_I32, [C.POINTER(IndexInfo), _P, _P, _P, _P, _I32, _P, C.c_int, C.POINTER(_P)]),
    "qv_index_set_nav": (_I32, [_P, _P, _P, _P, _I64, _I32, _I32]),
    "qv_index_get_info": (_I32, [_P, C.POINTER(IndexInfo)]),
    "qv_index_load_nav": (_I32, [_P, C.c_char_p]),
    "qv_index_neighbour_codes": (_I32, [_P, C.c_int32]),
    "qv_build_nav": (_I32, [_P, _P, _I64, _I32, _I32, C.POINTER(BuildParams), C.c_char_p]),
    "qv_index_close": (None, [_P]),
    "qv_search_opts_default": (None, [C.POINTER(SearchOpts)]),
    "qv_search": (_I32, [_P, _P, _I64, _I32, _I32, _I32, C.POINTER(SearchOpts), _P, _P, _P,
                         C.POINTER(SearchReport)]),
    "qv_search_noalloc": (_I32, [_P, _P, _I64, _I32, _I32, _I32, C.POINTER(SearchOpts), _P, _P, _P,
                                 C.POINTER(SearchReport)]),
    "qv_last_hops": (_I32, [_P, _P, _I64]),
    "qv_last_latencies": (_I32, [_P, _P, _I64]),
    "qv_last_error": (C.c_char_p, []),
    "qv_device_info": (_I32, [C.c_int, C.c_char_p, _I32, C.POINTER(_I32), C.POINTER(_I64)]),
    "qv_lut_build": (_I32, [_P, _P, _I64, _P, _P]),
    "qv_lut_build_raw": (_I32, [_P, _P, _P, _I32, _I32, _P, _I64, _P, _P, C.c_int]),
    "qv_adc_bench": (_I32, [_P, _I32, _P, _I64, _P, _I64, _I64, _I32, _P, _P, _P, C.c_int,
                            C.POINTER(C.c_float)]),
    "qv_gather_bench": (_I32, [_P, _I64, _P, _I64, _P, C.c_int, C.POINTER(C.c_float)]),
    "qv_stream_read_bench": (_I32, [_P, _I64, _P, C.c_int, C.POINTER(C.c_float)]),
    "qv_gather_rows_bench": (_I32, [_P, _I64, _I32, _P, _I64, _I32, _P, C.c_int, C.POINTER(C.c_float)]),
    "qv_fill_uniform_bytes": (_I32, [_P, _I64, C.c_uint64, C.c_int]),
    "qv_fill_uniform_ids": (_I32, [_P, _I64, _I64, C.c_uint64, C.c_int]),
    "qv_build_params_default": (None, [C.POINTER(BuildParams)]),
    "qv_build_index_cpu": (_I32, [_P, _I32, _I64, _I32, C.POINTER(BuildParams), C.c_char_p]),
    "qv_mixture_fill_host": (_I32, [C.POINTER(Mixture), _I64, _I64, _P]),
    "qv_mixture_fill_device": (_I32, [C.POINTER(Mixture), _I64, _I64, _P, C.c_int]),
    "qv_device_count": (_I32, [C.POINTER(_I32)]),
    "qv_gather_sweep_bench": (_I32, [_P, _I64, _I32, _P, _I64, _I64, _I32, _I32, _I32, _P, C.c_int,
                                     C.POINTER(C.c_float), C.POINTER(_I32)]),
    "qv_device_mem_info": (_I32, [C.c_int, C.POINTER(_I64), C.POINTER(_I64)]),
    "qv_build_index_gpu": (_I32, [_P, _I32, _I64, _I32, C.POINTER(BuildParams), C.c_int, C.POINTER(_P)]),
    "qv_index_save": (_I32, [_P, C.c_char_p]),
    "qv_index_copy_out": (_I32, [_P, _P, _P, _P, _P, _P]),
    "qv_ground_truth": (_I32, [_P, _I32, _I64, _I32, _P, _I64, _I32, _P, _P, C.c_int]),
    "qv_find_index_files": (_I32, [C.c_char_p, C.c_char_p, C.c_char_p, _I32]),
    "qv_read_layout": (_I32, [C.c_char_p, C.c_char_p, C.POINTER(IndexInfo)]),
    "qv_read_index_pages": (_I32, [C.c_char_p, _I64, _P]),
    "qv_dev_alloc": (_I32, [C.c_int, _I64, C.POINTER(_P)]),
    "qv_dev_free": (_I32, [_P]),
    "qv_dev_copy": (_I32, [_P, _P, _I64, _I32]),
    "qv_dev_clear": (_I32, [_P, _I64]),
}

_lib = None


def lib_path() -> Path:
    env = os.environ.get("QUIVER_HIP_LIB")
    return Path(env) if env else LIB_PATH


def load() -> C.CDLL:
    """Load libquiver_hip.so once; raise QuiverError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not path.is_file():
        raise QuiverError(
            f"libquiver_hip.so not found at {path}; build it with __graft_entry__.build() "
            "or `make -C quiver-ae_amd`"
        )
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    """Raise QuiverError carrying the library's thread-local message."""
    if rc != QV_OK:
        msg = load().qv_last_error()
        raise QuiverError(msg.decode() if msg else f"libquiver_hip error {rc}")


def default_search_opts() -> SearchOpts:
    o = SearchOpts()
    load().qv_search_opts_default(C.byref(o))
    return o


def default_build_params() -> BuildParams:
    p = BuildParams()
    load().qv_build_params_default(C.byref(p))
    return p


class DeviceBuffer:
    """Device allocation owned by the library's HIP runtime (freed on close/del)."""

    def __init__(self, nbytes: int, device: int = 0) -> None:
        self.nbytes = int(nbytes)
        self.device = device
        p = C.c_void_p()
        check(load().qv_dev_alloc(device, self.nbytes, C.byref(p)))
        self.ptr = p.value

    def upload(self, arr) -> "DeviceBuffer":
        import numpy as np

        a = np.ascontiguousarray(arr)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        check(load().qv_dev_copy(self.ptr, a.ctypes.data, a.nbytes, 0))
        return self

    def download(self, dtype, shape):
        import numpy as np

        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested more bytes than the device buffer holds")
        check(load().qv_dev_copy(out.ctypes.data, self.ptr, out.nbytes, 1))
        return out

    def clear(self) -> None:
        check(load().qv_dev_clear(self.ptr, self.nbytes))

    def close(self) -> None:
        if self.ptr:
            load().qv_dev_free(self.ptr)
            self.ptr = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def device_count() -> int:
    n = C.c_int32(0)
    check(load().qv_device_count(C.byref(n)))
    return n.value
