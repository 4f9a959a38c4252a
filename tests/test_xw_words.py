"""The packed exchange words of the sliced and layer-sequential kernels (plh_device.h): the helpers
are host functions too, so a host build of tests/xw_words_check.cpp checks their packed 16-bit
arithmetic exhaustively against the per-half definitions (CPU only; the GPU tests run them inside the
kernels, NaN rows included)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not found")
def test_exchange_word_helpers_match_their_definitions(tmp_path):
    exe = str(tmp_path / "xw_words_check")
    cmd = ["hipcc", "-x", "hip", "--cuda-host-only", "-O2", "-std=c++17", "-w",
           "-I", os.path.join(ROOT, "persistent_lstm_hip_amd", "csrc"),
           os.path.join(ROOT, "tests", "xw_words_check.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 mismatches" in out.stdout
