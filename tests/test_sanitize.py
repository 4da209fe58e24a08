"""The library's host-only C++ (file formats, CPU builder, C ABI helpers) and
the oracle built with AddressSanitizer + UndefinedBehaviorSanitizer and run on
small indexes and malformed inputs (CPU only; tests/cpp/host_sanitize_test.cpp).
A throwaway program with a heap overflow, built with the same flags, shows the
flags catch what they are meant to."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
CPP = HERE / "cpp"
FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


def test_host_code_under_asan_and_ubsan(tmp_path):
    subprocess.run(["make", "-C", str(CPP), "sanitize"], check=True, capture_output=True, timeout=600)
    r = subprocess.run([str(CPP / "_build" / "host_sanitize_test"), str(tmp_path / "work")],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "all checks passed" in r.stdout
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr


def test_the_flags_catch_a_heap_overflow(tmp_path):
    src = tmp_path / "overflow.cpp"
    src.write_text("#include <vector>\nint main(int c, char**) { std::vector<int> v(4); "
                   "return v.data()[3 + c]; }\n")
    exe = tmp_path / "overflow"
    subprocess.run(["g++", *FLAGS, str(src), "-o", str(exe)], check=True, capture_output=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr
