"""The host transfer runtime (si_host.cpp, with the session / control code of
si_api.cpp) under ThreadSanitizer and AddressSanitizer, on the CPU.

The library's host code is built with g++ against a test-only stand-in for
the HIP runtime (tests/csrc/hostsim: streams are worker threads, events are
generation counters completed in stream order, device memory is host memory,
and the layer kernels run as CPU tasks -- OpenSSL GCM, the oracle's codec,
the allocation-free entry's scratch ownership).  tests/csrc/hostsim/host_stress.cpp
then drives, concurrently: reload threads on their own streams through layer
groups (sealed on demand and ahead of demand, a record corrupted once and
repaired by the strict retry, one corrupted twice whose layer fails and whose
slot reads as zeros, bf16 and int4; a layer's causal groups merged into one
launch, sealed on demand or as one layer prefetch, with the tickets checked to
rise in the reference's K1 V1 K2 V2 order), D2H store batches spanning layers (bf16
and int8, batch_end racing the pool's verification, a corrupted record that
fails its batch), threads that end inside a layer group and inside a D2H
batch, a session destroyed while its prefetches are still being sealed, and a
destroy refused while another thread holds the session.  Every result is
checked against the host data, and the sanitizers stop at their first report.
A race planted in a copy of the driver (the cache read before the layer's
wait) is reported by this build, so a clean run means something."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOSTSIM = ROOT / "tests" / "csrc" / "hostsim"
OUT = ROOT / "tests" / "_build" / "hostsim"


def build(san: str) -> Path:
    subprocess.run(["make", "-s", "-C", str(HOSTSIM), f"SAN={san}", "-j2"], check=True, timeout=600)
    return OUT / f"host_stress_{san}"


@pytest.mark.parametrize("san,env,rounds", [
    ("thread", {"TSAN_OPTIONS": "halt_on_error=1 second_deadlock_stack=1"}, 3),
    ("address", {"ASAN_OPTIONS": "halt_on_error=1:detect_leaks=1"}, 3),
])
def test_host_runtime_under_sanitizer(san, env, rounds):
    exe = build(san)
    r = subprocess.run([str(exe), str(rounds)], capture_output=True, text=True, timeout=600,
                       env={**os.environ, **env})
    report = r.stdout + r.stderr
    assert "ThreadSanitizer" not in report and "AddressSanitizer" not in report and \
        "LeakSanitizer" not in report, report[-4000:]
    assert r.returncode == 0, report[-4000:]
    assert f"HOST_STRESS_OK rounds={rounds}" in r.stdout
