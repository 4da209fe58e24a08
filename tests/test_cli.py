"""quiver_search command line: flags, validation and error exits
(bin/quiver_search.cu:58-320, bin/common/cli_*.hpp).  The CPU cases fail
before any GPU work; the GPU case runs a search and checks the report lines
and result files."""
from __future__ import annotations

import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
CLI = ROOT / "quiver-ae_amd" / "bin" / "quiver_search"


def run(*args, timeout=120):
    if not CLI.is_file():
        pytest.fail(f"{CLI} not built")
    return subprocess.run([str(CLI), *map(str, args)], capture_output=True, text=True, timeout=timeout)


def test_help_and_required_flags():
    r = run("--help")
    assert r.returncode == 0 and "--index-dir" in r.stdout
    r = run("--query", "q.u8bin", "--data-type", "uint8")
    assert r.returncode == 1 and "--index-dir: required" in r.stderr


@pytest.mark.parametrize("flags,msg", [
    (["--pipe-width", "17"], "--pipe-width must be in [1, 16]"),
    (["--queries-per-block", "9"], "--queries-per-block must be in [1, 8]"),
    (["--num-blocks", "0"], "--num-blocks must be positive"),
    (["--early-exit-policy", "darth"], "invalid --early-exit-policy"),
    (["--num-blocks-list", "8,x"], "invalid integer in --num-blocks-list"),
    (["--bogus"], "Unknown argument"),
    (["--search-kernel", "fast"], "--search-kernel must be auto, lut or shared-pivots"),
    (["--graph-placement", "disk"], "--graph-placement must be hbm or host"),
])
def test_validation(tmp_path, flags, msg):
    r = run("--index-dir", tmp_path, "--query", "q.u8bin", "--data-type", "uint8", *flags)
    assert r.returncode == 1 and msg in r.stderr


@pytest.mark.parametrize("flags,msg", [
    (["--per-step-recall"], "--per-step-recall requires --ground-truth"),
    (["--per-step-recall", "--ground-truth", "gt.ibin"],
     "--per-step-recall currently requires pipe_width=1 and queries_per_block=1"),
    (["--per-step-recall", "--ground-truth", "gt.ibin", "--pipe-width", "1", "--queries-per-block", "2"],
     "--per-step-recall currently requires pipe_width=1 and queries_per_block=1"),
    (["--recall-threshold", "high"], "invalid float for --recall-threshold"),
])
def test_step_recall_validation(tmp_path, flags, msg):
    r = run("--index-dir", tmp_path, "--query", "q.u8bin", "--data-type", "uint8", *flags)
    assert r.returncode == 1 and msg in r.stderr


def test_spdk_requires_spdk_build(tmp_path):
    ssd = tmp_path / "ssds.txt"
    ssd.write_text("0000:01:00.0\n")
    r = run("--index-dir", tmp_path, "--query", "q.u8bin", "--data-type", "uint8", "--ssd-list-file", ssd)
    assert r.returncode == 1 and "built without SPDK support" in r.stderr


def test_missing_index_is_an_error(tmp_path):
    r = run("--index-dir", tmp_path / "none", "--query", "q.u8bin", "--data-type", "uint8")
    assert r.returncode == 1 and "does not exist" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("kernel,want", [(None, "lut"), ("shared-pivots", "shared-pivots")])
def test_cli_search_report_and_results(small_u8_index, tmp_path, kernel, want):
    import qv_oracle as O

    ix = small_u8_index
    q = ix["queries"][:100]
    qf = tmp_path / "q.u8bin"
    qf.write_bytes(struct.pack("<ii", *q.shape) + q.tobytes())
    gf = tmp_path / "gt.ibin"
    gf.write_bytes(struct.pack("<ii", 100, 10) + np.ascontiguousarray(ix["gt"][:100], np.int32).tobytes())
    print(f"[gpu] CLI search {ix['dir']}", flush=True)
    extra = ["--search-kernel", kernel] if kernel else []
    r = run("--index-dir", ix["dir"], "--query", qf, "--data-type", "uint8", "--ef-search", "64",
            "--repeat", "2", "--pipe-width", "1", "--ground-truth", gf, "--result-prefix", tmp_path / "res",
            "--early-exit-policy", "none", "--final-recall-csv", tmp_path / "r.csv", *extra)
    assert r.returncode == 0, r.stderr
    # 200 queries on 756 slots: auto takes the per-query-LUT kernel
    assert f"[Quiver] search_kernel={want}" in r.stdout
    assert "QPS:" in r.stdout and "QueryLatency(ms): avg=" in r.stdout and "Recall @ 10:" in r.stdout
    ids = np.fromfile(tmp_path / "res_ids.bin", dtype="<i4")
    n, k = ids[:2]
    assert (n, k) == (200, 10)
    ids = ids[2:].reshape(200, 10)
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, _, _, _ = O.search(host, q.astype(np.float32), 10, 64, early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids[:100], oids)
    np.testing.assert_array_equal(ids[100:], oids)   # --repeat 2 repeats the set
    line = [s for s in r.stdout.splitlines() if s.startswith("Recall @ 10:")][0]
    assert abs(float(line.split(":")[1]) - O.recall(oids, ix["gt"][:100], 10)) < 1e-6
    assert (tmp_path / "r.csv").read_text().startswith("query_id,gt_query_id,hits,recall")


@pytest.mark.gpu
def test_cli_per_step_recall_matches_oracle(small_u8_index, tmp_path):
    """--per-step-recall: the step CSV and summary lines (search.cu:112-153)
    against the oracle's per-step recall on the same queries."""
    import qv_oracle as O

    ix = small_u8_index
    q = ix["queries"][:120]
    qf = tmp_path / "q.u8bin"
    qf.write_bytes(struct.pack("<ii", *q.shape) + q.tobytes())
    gt = np.ascontiguousarray(ix["gt"][:120], np.int32)
    gf = tmp_path / "gt.ibin"
    gf.write_bytes(struct.pack("<ii", *gt.shape) + gt.tobytes())
    csv = tmp_path / "steps.csv"
    print("[gpu] CLI --per-step-recall", flush=True)
    r = run("--index-dir", ix["dir"], "--query", qf, "--data-type", "uint8", "--ef-search", "96",
            "--repeat", "1", "--pipe-width", "1", "--ground-truth", gf, "--early-exit-policy", "none",
            "--per-step-recall", "--recall-threshold", "0.8", "--step-recall-csv", csv)
    assert r.returncode == 0, r.stderr
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    _, _, _, _, step, hits = O.search(host, q.astype(np.float32), 10, 96, early_exit=O.EXIT_NONE,
                                      step_recall=(gt, O.required_hits(0.8, 10)))
    rows = [line.split(",") for line in csv.read_text().splitlines()]
    assert rows[0] == ["query_id", "step", "hits", "recall", "reached"]
    got = np.array([[int(x[1]), int(x[2]), int(x[4])] for x in rows[1:]])
    np.testing.assert_array_equal(got[:, 0], step)
    np.testing.assert_array_equal(got[:, 1], hits)
    np.testing.assert_array_equal(got[:, 2], (step >= 0).astype(int))
    reached = int((step >= 0).sum())
    assert f"[Quiver] Step recall reached={reached} unreached={120 - reached} threshold=0.8 required_hits=8" in r.stdout
    assert "[Quiver] per-step recall enabled: threshold=0.8" in r.stdout


@pytest.mark.gpu
def test_cli_default_slots_fill_the_gpu(small_u8_index, tmp_path):
    """Without --num-blocks the whole GPU holds query slots: a batch larger
    than the per-query-LUT kernel's resident slots runs the shared-pivot
    kernel, with the same results as an explicit small slot count."""
    ix = small_u8_index
    q = ix["queries"][:200]
    qf = tmp_path / "q.u8bin"
    qf.write_bytes(struct.pack("<ii", *q.shape) + q.tobytes())
    common = ["--index-dir", ix["dir"], "--query", qf, "--data-type", "uint8", "--ef-search", "64",
              "--repeat", "12", "--pipe-width", "1", "--early-exit-policy", "none"]
    print("[gpu] CLI default slots, 2400 queries", flush=True)
    r = run(*common, "--result-prefix", tmp_path / "a")
    assert r.returncode == 0, r.stderr
    assert "[Quiver] search_kernel=shared-pivots" in r.stdout
    slots = int(r.stdout.split("Runtime Params:\n  num_blocks=")[1].split()[0])
    assert slots > 1024
    print("[gpu] CLI --num-blocks 756, 2400 queries", flush=True)
    r2 = run(*common, "--num-blocks", "756", "--result-prefix", tmp_path / "b")
    assert r2.returncode == 0, r2.stderr
    slots2 = int(r2.stdout.split("Runtime Params:\n  num_blocks=")[1].split()[0])
    assert 756 <= slots2 < 756 + 16  # a launch may round the slots up to whole workgroups
    a = np.fromfile(tmp_path / "a_ids.bin", dtype="<i4")
    b = np.fromfile(tmp_path / "b_ids.bin", dtype="<i4")
    np.testing.assert_array_equal(a, b)


def test_static_batches_without_num_blocks_parses(tmp_path):
    """--static-batches with --num-blocks unset is accepted by the parser and
    reaches the index (an ordinary error for a missing one, not a signal)."""
    r = run("--index-dir", tmp_path / "none", "--query", "q.u8bin", "--data-type", "uint8", "--static-batches")
    assert r.returncode == 1 and "does not exist" in r.stderr


@pytest.mark.gpu
def test_cli_static_batches_fill_the_gpu(small_u8_index, tmp_path):
    """--static-batches without --num-blocks: batches of the slots that fill
    the GPU, reported after the search; ids equal the oracle's."""
    import qv_oracle as O

    ix = small_u8_index
    q = ix["queries"][:300]
    qf = tmp_path / "q.u8bin"
    qf.write_bytes(struct.pack("<ii", *q.shape) + q.tobytes())
    print("[gpu] CLI --static-batches without --num-blocks", flush=True)
    r = run("--index-dir", ix["dir"], "--query", qf, "--data-type", "uint8", "--ef-search", "64", "--repeat", "1",
            "--pipe-width", "1", "--early-exit-policy", "none", "--static-batches",
            "--result-prefix", tmp_path / "s")
    assert r.returncode == 0, r.stderr
    line = [s for s in r.stdout.splitlines() if s.startswith("[Quiver] StaticBatch:")]
    assert line and "total 300 queries" in line[0], r.stdout
    ids = np.fromfile(tmp_path / "s_ids.bin", dtype="<i4")[2:].reshape(300, 10)
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, _, _, _ = O.search(host, q.astype(np.float32), 10, 64, early_exit=O.EXIT_NONE)
    np.testing.assert_array_equal(ids, oids)


@pytest.mark.gpu
def test_cli_wide_topk_and_deep_beam(small_u8_index, tmp_path):
    """--topk 100 --ef-search 1500 (entries past the 64th top-k in LDS, a beam
    of 32 positions per lane): the result files hold the oracle's ids and
    distances for every repetition of the query set."""
    import qv_oracle as O

    ix = small_u8_index
    q = ix["queries"][:40]
    qf = tmp_path / "q.u8bin"
    qf.write_bytes(struct.pack("<ii", *q.shape) + q.tobytes())
    print("[gpu] CLI --topk 100 --ef-search 1500 --repeat 2", flush=True)
    r = run("--index-dir", ix["dir"], "--query", qf, "--data-type", "uint8", "--topk", "100", "--ef-search", "1500",
            "--repeat", "2", "--pipe-width", "2", "--early-exit-policy", "gpruning", "--result-prefix",
            tmp_path / "w")
    assert r.returncode == 0, r.stderr
    ids = np.fromfile(tmp_path / "w_ids.bin", dtype="<i4")
    dists = np.fromfile(tmp_path / "w_distances.bin", dtype="<f4")
    assert tuple(ids[:2]) == (80, 100) and tuple(dists[:2].view("<i4")) == (80, 100)
    host = O.HostIndex.from_files(ix["dir"], "uint8")
    oids, odists, _, _ = O.search(host, q.astype(np.float32), 100, 1500, pipe_width=2, early_exit=O.EXIT_GPRUNING)
    np.testing.assert_array_equal(ids[2:].reshape(80, 100), np.concatenate([oids, oids]))
    np.testing.assert_array_equal(dists[2:].reshape(80, 100), np.concatenate([odists, odists]))
