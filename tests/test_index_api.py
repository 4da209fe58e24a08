"""Contract of IndexQuiver's external-engine path and of its argument checks.

What is pinned is the binding contract of python/quiver/index.py:27-264 (the
behaviour python/tests/test_index.py:13-113 exercises): the engine's command
line, the int32-headed query and result files, how SSD lists and SPDK_BASE_LBA
reach the engine, and the errors for a failing, hanging or misbehaving engine.
The fake engine below is this project's own: it logs what it was given and
derives every result from the query values it read, so a query that arrives
altered, in the wrong element type or in the wrong order fails a test.  CPU only.
"""
from __future__ import annotations

import json
import stat
import sys
from pathlib import Path

import numpy as np
import pytest

from quiver import IndexQuiver, QuiverError

ENGINE = r'''
import json, os, sys, time
import numpy as np

argv = sys.argv[1:]
opts = {}
i = 0
while i < len(argv):
    if argv[i].startswith("--") and i + 1 < len(argv) and not argv[i + 1].startswith("--"):
        opts[argv[i]] = argv[i + 1]
        i += 2
    else:
        opts[argv[i]] = None
        i += 1
log = os.environ.get("ENGINE_LOG")
ssds = None
if "--ssd-list-file" in opts:
    ssds = open(opts["--ssd-list-file"]).read().splitlines()
if log:
    json.dump({"argv": argv, "opts": opts, "ssds": ssds,
               "lba": os.environ.get("SPDK_BASE_LBA"), "marker": os.environ.get("ENGINE_MARKER")},
              open(log, "w"))
mode = os.environ.get("ENGINE_MODE", "ok")
if mode == "fail":
    sys.stderr.write("  graph pages unreadable  \n")
    sys.exit(5)
if mode == "fail_stdout":
    print("only stdout says why")
    sys.exit(9)
if mode == "hang":
    time.sleep(60)
elem = {"float": "<f4", "uint8": "u1", "int8": "i1"}[opts["--data-type"]]
raw = open(opts["--query"], "rb").read()
rows, cols = np.frombuffer(raw, "<i4", 2)
q = np.frombuffer(raw[8:], elem).reshape(rows, cols).astype(np.float64)
k = int(opts["--topk"])
ids = (np.arange(rows)[:, None] * 100 + np.arange(k)[None, :]).astype("<i4")
dists = (q.sum(axis=1)[:, None] + np.arange(k)[None, :] * 0.5).astype("<f4")
prefix = opts["--result-prefix"]
if mode == "skip_dists":
    outputs = (("_ids.bin", ids),)
else:
    outputs = (("_ids.bin", ids), ("_distances.bin", dists))
for suffix, arr in outputs:
    body = arr.tobytes()
    head = np.array([rows, k], "<i4").tobytes()
    if mode == "short_header" and suffix == "_ids.bin":
        head, body = head[:5], b""
    if mode == "negative" and suffix == "_ids.bin":
        head = np.array([-1, k], "<i4").tobytes()
    if mode == "truncated" and suffix == "_distances.bin":
        body = body[:-3]
    if mode == "wide" and suffix == "_ids.bin":
        head = np.array([rows, k + 1], "<i4").tobytes()
        body = np.zeros((rows, k + 1), "<i4").tobytes()
    open(prefix + suffix, "wb").write(head + body)
'''


@pytest.fixture()
def engine(tmp_path: Path) -> Path:
    path = tmp_path / "engine" / "quiver_search"
    path.parent.mkdir()
    path.write_text(f"#!{sys.executable}\n{ENGINE}", encoding="utf-8")
    path.chmod(path.stat().st_mode | stat.S_IXUSR)
    return path


@pytest.fixture()
def index_dir(tmp_path: Path) -> Path:
    d = tmp_path / "idx"
    d.mkdir()
    return d


def _logged(tmp_path: Path, index: IndexQuiver, queries, **kw):
    log = tmp_path / "engine.json"
    index.env["ENGINE_LOG"] = str(log)
    out = index.search(queries, **kw)
    return out, json.loads(log.read_text())


def test_command_line_carries_every_setting(tmp_path: Path, engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, data_type="uint8", binary=engine, memory_backend="mmap", num_blocks=432,
                        queries_per_block=2, pipe_width=4, poll_threads=3, runners_per_ssd=2)
    (_, _), seen = _logged(tmp_path, index, np.full((2, 8), 7, np.uint8), topk=5, ef_search=77,
                           early_exit_policy="none", extra_args=["--skip-nav"])
    opts = seen["opts"]
    expect = {"--index-dir": str(index_dir.resolve()), "--data-type": "uint8", "--topk": "5",
              "--ef-search": "77", "--repeat": "1", "--num-blocks": "432", "--queries-per-block": "2",
              "--pipe-width": "4", "--poll-threads": "3", "--runners-per-ssd": "2",
              "--memory-backend": "mmap", "--early-exit-policy": "none"}
    for flag, value in expect.items():
        assert opts[flag] == value, flag
    assert Path(opts["--query"]).name == "queries.u8bin"
    assert Path(opts["--result-prefix"]).name == "result"
    assert "--ssd-list-file" not in opts
    assert seen["argv"][-1] == "--skip-nav"  # extra arguments come last, verbatim
    assert seen["lba"] is None


def test_defaults_on_the_command_line(tmp_path: Path, engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, binary=engine)
    (ids, _), seen = _logged(tmp_path, index, np.ones((1, 3), np.float32))
    opts = seen["opts"]
    assert (opts["--data-type"], opts["--topk"], opts["--ef-search"]) == ("float", "10", "50")
    assert (opts["--num-blocks"], opts["--pipe-width"], opts["--queries-per-block"]) == ("756", "2", "1")
    assert (opts["--poll-threads"], opts["--runners-per-ssd"]) == ("6", "1")
    assert (opts["--memory-backend"], opts["--early-exit-policy"]) == ("heap", "gpruning")
    assert Path(opts["--query"]).name == "queries.fbin"
    assert ids.shape == (1, 10)


@pytest.mark.parametrize("data_type,sent,suffix", [
    ("float32", np.array([[0.25, -1.5, 3.0]]), ".fbin"),
    ("float", np.array([[0.25, -1.5, 3.0]], np.float32), ".fbin"),
    ("uint8", np.array([[1, 2, 250]]), ".u8bin"),
    ("int8", np.array([[-5, 2, 100]]), ".i8bin"),
])
def test_queries_reach_the_engine_as_the_index_type(tmp_path: Path, engine: Path, index_dir: Path,
                                                    data_type, sent, suffix) -> None:
    index = IndexQuiver(index_dir, data_type=data_type, binary=engine)
    (ids, dists), seen = _logged(tmp_path, index, sent, topk=3)
    assert Path(seen["opts"]["--query"]).suffix == suffix
    # the engine sums each query row: the values came through unchanged
    np.testing.assert_array_equal(dists[:, 0], np.asarray(sent, np.float64).sum(axis=1).astype(np.float32))


def test_result_files_become_arrays(engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, data_type="float32", binary=engine)
    q = np.arange(12, dtype=np.float64).reshape(3, 4)
    ids, dists = index.search(q, topk=4)
    assert ids.dtype == np.dtype("<i4") and dists.dtype == np.dtype("<f4")
    assert ids.shape == dists.shape == (3, 4)
    np.testing.assert_array_equal(ids[2], [200, 201, 202, 203])
    np.testing.assert_array_equal(dists[:, 1], q.sum(axis=1) + 0.5)


def test_single_vector_is_one_query(engine: Path, index_dir: Path) -> None:
    ids, dists = IndexQuiver(index_dir, binary=engine).search(np.array([1.0, 2.0, 4.0]), topk=2)
    assert ids.shape == (1, 2)
    assert dists[0, 0] == 7.0


def test_ssd_addresses_written_to_a_list_file(tmp_path: Path, engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, binary=engine, ssds=[" 0000:41:00.0", "0000:42:00.0 ", "0000:43:00.0"],
                        spdk_base_lba=2048)
    assert index.num_ssds == 3
    _, seen = _logged(tmp_path, index, np.ones((1, 2), np.float32))
    assert seen["ssds"] == ["0000:41:00.0", "0000:42:00.0", "0000:43:00.0"]
    assert seen["lba"] == "2048"


def test_ssd_list_file_passed_through(tmp_path: Path, engine: Path, index_dir: Path) -> None:
    listing = tmp_path / "mine.txt"
    listing.write_text("# striped pair\n0000:81:00.0\n\n   \n0000:82:00.0\n  # spare\n", encoding="ascii")
    index = IndexQuiver(index_dir, binary=engine, ssd_list_file=listing)
    assert index.num_ssds == 2  # comments and blank lines are not SSDs
    _, seen = _logged(tmp_path, index, np.ones((1, 2), np.float32))
    assert seen["opts"]["--ssd-list-file"] == str(listing.resolve())


def test_env_reaches_the_engine(tmp_path: Path, engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, binary=engine, env={"ENGINE_MARKER": "blue"})
    _, seen = _logged(tmp_path, index, np.ones((1, 2), np.float32))
    assert seen["marker"] == "blue"


def test_binary_from_environment(monkeypatch, engine: Path, index_dir: Path) -> None:
    monkeypatch.setenv("QUIVER_BINARY", str(engine))
    index = IndexQuiver(index_dir)
    assert index.binary == engine.resolve()
    assert index.search(np.ones((2, 2), np.float32), topk=1)[0].shape == (2, 1)


@pytest.mark.parametrize("mode,message", [
    ("fail", "quiver_search exited with code 5: graph pages unreadable$"),
    ("fail_stdout", "quiver_search exited with code 9: only stdout says why"),
    ("skip_dists", "quiver_search did not create result_distances.bin"),
    ("short_header", "invalid result header in .*result_ids.bin"),
    ("negative", "invalid result dimensions in .*result_ids.bin"),
    ("truncated", "truncated result data in .*result_distances.bin"),
    ("wide", r"unexpected result shape: ids=\(2, 4\), distances=\(2, 3\), expected=\(2, 3\)"),
])
def test_engine_misbehaviour_is_quiver_error(engine: Path, index_dir: Path, mode, message) -> None:
    index = IndexQuiver(index_dir, binary=engine, env={"ENGINE_MODE": mode})
    with pytest.raises(QuiverError, match=message):
        index.search(np.ones((2, 2), np.float32), topk=3)


def test_engine_timeout(engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, binary=engine, env={"ENGINE_MODE": "hang"})
    with pytest.raises(QuiverError, match="exceeded the 0.2 second timeout"):
        index.search(np.ones((1, 2), np.float32), timeout=0.2)


def test_constructor_validation(tmp_path: Path, engine: Path, index_dir: Path) -> None:
    listing = tmp_path / "l.txt"
    listing.write_text("0000:01:00.0\n")
    cases = [
        (dict(index_dir=tmp_path / "absent"), ValueError, "index_dir is not a directory"),
        (dict(data_type="float16"), ValueError, "data_type must be float32, float, uint8, or int8"),
        (dict(ssds=["0000:01:00.0"], ssd_list_file=listing), ValueError, "either ssds or ssd_list_file"),
        (dict(ssds=["0000:01:00.0", "  "]), ValueError, "SSD PCI addresses must not be empty"),
        (dict(ssd_list_file=tmp_path / "nope.txt"), ValueError, "ssd_list_file does not exist"),
        (dict(spdk_base_lba=-1), ValueError, "spdk_base_lba must be non-negative"),
        (dict(memory_backend="disk"), ValueError, "memory_backend must be heap or mmap"),
        (dict(graph_placement="disk"), ValueError, "graph_placement must be hbm or host"),
        (dict(search_kernel="fast"), ValueError, "search_kernel must be"),
        (dict(num_blocks=0), ValueError, "num_blocks must be positive"),
        (dict(queries_per_block=-2), ValueError, "queries_per_block must be positive"),
        (dict(pipe_width=0), ValueError, "pipe_width must be positive"),
        (dict(poll_threads=0), ValueError, "poll_threads must be positive"),
        (dict(runners_per_ssd=0), ValueError, "runners_per_ssd must be positive"),
        (dict(binary=tmp_path / "no_engine"), QuiverError, "quiver_search executable not found"),
        (dict(binary=listing), QuiverError, "quiver_search executable not found"),  # not executable
    ]
    for kw, err, message in cases:
        args = {"index_dir": index_dir, "binary": engine, **kw}
        with pytest.raises(err, match=message):
            IndexQuiver(args.pop("index_dir"), **args)


def test_search_validation(engine: Path, index_dir: Path) -> None:
    index = IndexQuiver(index_dir, binary=engine)
    cases = [
        (dict(topk=0), "topk must be positive"),
        (dict(ef_search=-1), "ef_search must be positive"),
        (dict(early_exit_policy="darth"), "early_exit_policy must be gpruning or none"),
        (dict(timeout=0), "timeout must be positive"),
    ]
    for kw, message in cases:
        with pytest.raises(ValueError, match=message):
            index.search(np.ones((1, 2), np.float32), **kw)
    for bad in (np.ones((0, 4)), np.ones((3, 0)), np.ones((2, 2, 2)), np.float32(1.0)):
        with pytest.raises(ValueError, match="non-empty 1D or 2D"):
            index.search(bad)


def test_in_process_engine_refuses_ssds_and_reports_missing_index(index_dir: Path) -> None:
    with pytest.raises(QuiverError, match="without SPDK support"):
        IndexQuiver(index_dir, data_type="uint8", ssds=["0000:01:00.0"]).search(np.ones((1, 4), np.uint8))
    with pytest.raises(QuiverError, match="extra_args other than --skip-nav"):
        IndexQuiver(index_dir, data_type="uint8").search(np.ones((1, 4), np.uint8), extra_args=["--x"])
    with pytest.raises(QuiverError, match=r"No \*_disk.index"):
        IndexQuiver(index_dir, data_type="uint8").search(np.ones((1, 4), np.uint8))


def test_num_blocks_default_fills_the_gpu_in_process(index_dir: Path) -> None:
    # the in-process engine opens the index only at the first search, so this
    # runs without a GPU: unset, num_blocks is 0 (the whole device)
    assert IndexQuiver(index_dir, data_type="uint8").num_blocks == 0
    assert IndexQuiver(index_dir, data_type="uint8", num_blocks=756).num_blocks == 756
    with pytest.raises(ValueError, match="num_blocks must be positive"):
        IndexQuiver(index_dir, data_type="uint8", num_blocks=0)
