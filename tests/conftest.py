"""Shared fixtures: import paths, the `gpu` marker, small CPU-built indexes."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "quiver-ae_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X")


@pytest.fixture(scope="session")
def small_u8_index(tmp_path_factory):
    """20k-point uint8 mixture index, R=32, M=32, plus queries and ground truth."""
    import quiver
    import qv_oracle as O

    d = tmp_path_factory.mktemp("u8idx")
    base = quiver.mixture(20000, 128, num_centers=64, seed=7)
    queries = quiver.mixture(300, 128, num_centers=64, seed=7, first_row=10**7)
    quiver.build_index(base, d / "small", R=32, L=64, num_chunks=32, threads=0)
    gt, _ = O.ground_truth(base, queries, 10)
    return {"dir": d, "base": base, "queries": queries, "gt": gt, "dtype": "uint8"}


@pytest.fixture(scope="session")
def small_f32_index(tmp_path_factory):
    """8k-point normalised float mixture index, d=96, R=64, M=48 (2 dims per chunk)."""
    import quiver
    import qv_oracle as O

    d = tmp_path_factory.mktemp("f32idx")
    base = quiver.mixture(8000, 96, data_type="float", num_centers=64, seed=11, sigma=1.0)
    queries = quiver.mixture(200, 96, data_type="float", num_centers=64, seed=11, sigma=1.0,
                             first_row=10**7)
    quiver.build_index(base, d / "flt", R=64, L=80, num_chunks=48, threads=0)
    gt, _ = O.ground_truth(base, queries, 10)
    return {"dir": d, "base": base, "queries": queries, "gt": gt, "dtype": "float"}


def gpu_available() -> bool:
    try:
        from quiver import _lib

        return _lib.device_count() > 0
    except Exception:
        return False
