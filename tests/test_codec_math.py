"""The codec quantiser's rounding helpers (secure_infer_amd/csrc/si_codec_math.h),
checked as compiled code rather than restated:

* CPU: recip_refine / div_rn against IEEE division on ~9e7 cases, incl.
  quotients next to k + 0.5 ties (tests/csrc/codec_div_check.hip, host-only
  build of the same header);
* GPU: v_cvt_pk_u8_f32 (int8 / int4 insertion) and v_cvt_pk_bf16_f32 against
  integer round-to-nearest-even references over all 2^32 float patterns
  (tests/csrc/codec_cvt_sweep.hip, built by build() into tests/_build)."""
import ctypes as ct
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "secure_infer_amd" / "csrc"


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    pytest.skip("hipcc not available")


def test_division_matches_ieee(tmp_path):
    exe = tmp_path / "codec_div_check"
    subprocess.run([_hipcc(), "--cuda-host-only", "-x", "hip", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I", str(CSRC), str(ROOT / "tests" / "csrc" / "codec_div_check.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    fields = out.stdout.split()
    stats = dict(zip(fields[0::2], map(int, fields[1::2])))
    assert stats["bad"] == 0 and stats["cases"] > 50_000_000
    assert stats["naive_differs"] > 0  # the cases do separate a*RN(1/s) from RN(a/s)


@pytest.mark.gpu
def test_packed_conversions_every_float():
    import torch
    lib_path = ROOT / "tests" / "_build" / "libsi_selftest.so"
    assert lib_path.exists(), "run build() first"
    lib = ct.CDLL(str(lib_path))
    lib.si_selftest_cvt_sweep.argtypes = [ct.c_void_p, ct.c_void_p]
    lib.si_selftest_cvt_sweep.restype = ct.c_int
    counts = torch.zeros(4, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    assert lib.si_selftest_cvt_sweep(ct.c_void_p(stream.cuda_stream), ct.c_void_p(counts.data_ptr())) == 0
    torch.cuda.synchronize()
    bad8, bad4, badbf, seen = counts.tolist()
    assert seen == 1 << 32
    assert (bad8, bad4, badbf) == (0, 0, 0)
