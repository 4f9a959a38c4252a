"""Build recipe of the native library (hipcc, gfx950 only).

    python -m persistent_lstm_hip_amd.build        # -> persistent_lstm_hip_amd/lib/libpersistent_lstm_hip.so

The library exposes the C ABI declared in include/persistent_lstm_hip.h.  It is built in-tree so
that the .so travels with the source tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libpersistent_lstm_hip.so")
BENCH_PATH = os.path.join(LIB_DIR, "plh_bench")
SOURCES = ["plh_wavefront.hip", "plh_sliced.hip", "plh_rec.hip", "plh_gemm.hip", "plh_pack.hip", "plh_launch.hip",
           "plh_probe.hip", "plh_capi.hip"]
HEADERS = ["plh_internal.h", os.path.join("..", "..", "include", "persistent_lstm_hip.h")]

ARCH = "gfx950"
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-shared",
    # Keep packed-FP32 VALU ops out of the generated code (v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]
# Only the HIP runtime (hipcc links it); every kernel is in csrc/, no vendor math library.
LINK_FLAGS: list = []


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the native library needs ROCm's hipcc")
    return path


def build(verbose: bool = False) -> str:
    """Compile every source for gfx950 and link the shared library.  Always recompiles."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc()] + HIPCC_FLAGS + [os.path.join(CSRC, s) for s in SOURCES] + LINK_FLAGS + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB_PATH)
    # Native driver of the C ABI (profiling target and integration example), linked to the library.
    # (plh_issue_probe.hip: a developer probe kernel of plh_bench --issue, not part of the library.)
    cmd = [hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-Wno-unused-command-line-argument", os.path.join(CSRC, "plh_bench_main.cpp"),
           os.path.join(CSRC, "plh_issue_probe.hip"), "-L" + LIB_DIR, "-lpersistent_lstm_hip", "-Wl,-rpath,$ORIGIN",
           "-o", BENCH_PATH + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc (plh_bench) failed ({proc.returncode}):\n{proc.stdout}")
    os.replace(BENCH_PATH + ".tmp", BENCH_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
