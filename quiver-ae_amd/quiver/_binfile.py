"""int32-headed matrix files exchanged with an external ``quiver_search``.

Layout (bin/common/data_io.hpp:29-51, 116-140): little-endian int32 rows, int32
columns, then rows x columns elements, row-major.  The query file the engine
reads and the ``<prefix>_ids.bin`` / ``<prefix>_distances.bin`` files it writes
all use it.  Errors carry the messages of the reference binding
(python/quiver/index.py:222-236), since callers match on them.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from ._lib import QuiverError

_HEADER = np.dtype([("rows", "<i4"), ("cols", "<i4")])


def write_matrix(path: Path, matrix: np.ndarray) -> None:
    """Writes a 2-D array with its (rows, cols) header."""
    header = np.array([(matrix.shape[0], matrix.shape[1])], dtype=_HEADER)
    with open(path, "wb") as f:
        header.tofile(f)
        np.ascontiguousarray(matrix).tofile(f)


def read_matrix(path: Path, dtype: str) -> np.ndarray:
    """Reads a result matrix of little-endian `dtype` elements; raises
    QuiverError when the file is missing, its header is short or negative, or
    the body does not hold exactly rows x cols elements."""
    try:
        raw = path.read_bytes()
    except FileNotFoundError:
        raise QuiverError(f"quiver_search did not create {path.name}") from None
    if len(raw) < _HEADER.itemsize:
        raise QuiverError(f"invalid result header in {path}")
    head = np.frombuffer(raw, dtype=_HEADER, count=1)[0]
    rows, cols = int(head["rows"]), int(head["cols"])
    if rows < 0 or cols < 0:
        raise QuiverError(f"invalid result dimensions in {path}")
    elem = np.dtype(dtype).newbyteorder("<")
    body = memoryview(raw)[_HEADER.itemsize:]
    if len(body) // elem.itemsize != rows * cols:
        raise QuiverError(f"truncated result data in {path}")
    values = np.frombuffer(body, dtype=elem, count=rows * cols)
    return values.astype(elem.newbyteorder("="), copy=True).reshape(rows, cols)
