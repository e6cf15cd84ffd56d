"""Builds libsecure_infer.so (HIP for gfx950) in-tree with hipcc, and the
GPU self-test library the tests load (tests/_build/libsi_selftest.so: the
sweep of the codec's packed conversions over every float pattern)."""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
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
    """Each source compiled on its own (in parallel: the record kernel's
    source alone takes about two minutes), then linked."""
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    compile_flags = [f for f in FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="si_build_") as d:
        objs = [Path(d) / (Path(s).stem + ".o") for s in SOURCES]
        cmds = [[hipcc(), *compile_flags, "-I", str(ROOT / "include"), "-I", str(CSRC), "-c", "-o", str(o),
                 str(CSRC / s)] for s, o in zip(SOURCES, objs)]
        for c in cmds:
            if verbose:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
            for r in list(ex.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds)):
                if r.returncode != 0:
                    sys.stderr.write(r.stdout + r.stderr)
                    raise subprocess.CalledProcessError(r.returncode, r.args)
        link_flags = [f for f in FLAGS if not f.startswith("-amdgpu-") and f != "-mllvm"]
        cmd = [hipcc(), *link_flags, "-o", str(tmp), *[str(o) for o in objs], *LIBS]
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
