"""Builds libsecure_infer.so (HIP for gfx950) in-tree with hipcc, and the
GPU self-test library the tests load (tests/_build/libsi_selftest.so: the
sweep of the codec's packed conversions over every float pattern)."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_lib" / "libsecure_infer.so"
SELFTEST_SRC = ROOT / "tests" / "csrc" / "codec_cvt_sweep.hip"
SELFTEST_OUT = ROOT / "tests" / "_build" / "libsi_selftest.so"

SOURCES = ["si_gcm.hip", "si_codec.hip", "si_agree.hip", "si_api.cpp", "si_host.cpp"]
LIBS = ["-lcrypto", "-lpthread"]

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    # packed FP32 ops stay off for every HIP source on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # gfx950 kernel-argument preload: the first kernel argument words (the
    # key-context pointer) arrive in SGPRs, so the set-up's table fills go
    # out before the kernel-argument load returns (A/B on MI355X: -0.5 to
    # -1 % per layer on every workload)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    return "hipcc"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, "-I", str(ROOT / "include"), "-I", str(CSRC), "-o", str(tmp),
           *[str(CSRC / s) for s in SOURCES], *LIBS]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    if SELFTEST_SRC.exists():
        SELFTEST_OUT.parent.mkdir(parents=True, exist_ok=True)
        tmp = SELFTEST_OUT.with_suffix(".so.tmp")
        cmd = [hipcc(), *FLAGS, "-I", str(CSRC), "-o", str(tmp), str(SELFTEST_SRC)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp, SELFTEST_OUT)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(OUT)
