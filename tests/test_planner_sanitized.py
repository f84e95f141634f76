"""The slot planner's host code under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU): random create / plan / plan_each / peek /
note_token sequences, invalid keys and pins included, over many planner
shapes and both policies (the reference builds its planner with warnings as
errors only, native/Makefile:2; this adds a memory-safety check of ours)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_planner_is_clean_under_address_and_ub_sanitizers(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "planner_fuzz"
    cmd = [gxx, "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", f"-I{ROOT / 'include'}", "-x", "c++",
           str(ROOT / "tests" / "native" / "planner_fuzz.c"), "-x", "none",
           str(ROOT / "locali_amd" / "csrc" / "slot_planner.cpp"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    if build.returncode != 0 and "sanitize" in build.stderr:
        pytest.skip("sanitizer runtime not available: " + build.stderr[-200:])
    assert build.returncode == 0, build.stderr[-2000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=240)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "fuzz ok" in run.stdout
