"""The device caching allocator's bookkeeping (lucid_amd/csrc/lq_block_cache.h), compiled
for the host with g++ and driven with fake completion markers (no GPU): a freed block is
reused on its own stream at once and on another stream only after the marker recorded at
its free completes."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_block_cache_bookkeeping(tmp_path):
    exe = tmp_path / "block_cache_check"
    src = os.path.join(ROOT, "tests", "native", "block_cache_check.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    "-I", os.path.join(ROOT, "lucid_amd", "csrc"), src, "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok"
