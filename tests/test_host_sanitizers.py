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
wait) is reported by the sanitizer build, so a clean run means something."""
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


@pytest.mark.parametrize("san,env,rounds,ledger", [
    ("thread", {"TSAN_OPTIONS": "halt_on_error=1 second_deadlock_stack=1"}, 3, False),
    ("address", {"ASAN_OPTIONS": "halt_on_error=1:detect_leaks=1"}, 3, False),
    # the H2D ledger in records mode on: its rows are retired as ring slots
    # are reused, from every thread that launches
    ("thread", {"TSAN_OPTIONS": "halt_on_error=1 second_deadlock_stack=1",
                "SECURE_INFER_H2D_PROFILE_RECORDS": "1"}, 2, True),
], ids=["thread", "address", "thread_ledger"])
def test_host_runtime_under_sanitizer(san, env, rounds, ledger, tmp_path):
    exe = build(san)
    env = dict(env)
    if ledger:
        env["SECURE_INFER_H2D_PROFILE"] = str(tmp_path / "ledger.csv")
    r = subprocess.run([str(exe), str(rounds)], capture_output=True, text=True, timeout=600,
                       env={**os.environ, **env})
    report = r.stdout + r.stderr
    assert "ThreadSanitizer" not in report and "AddressSanitizer" not in report and \
        "LeakSanitizer" not in report, report[-4000:]
    assert r.returncode == 0, report[-4000:]
    assert f"HOST_STRESS_OK rounds={rounds}" in r.stdout
    if ledger:
        lines = (tmp_path / "ledger.csv").read_text().splitlines()
        assert lines[0].startswith("direction,bytes,aligned_bytes,total_us,cpu_crypto_us") and len(lines) > 1
        assert all(l.startswith("H2D,") and len(l.split(",")) == 16 for l in lines[1:])


@pytest.mark.parametrize("abort", [False, True], ids=["batch_fails", "process_aborts"])
def test_d2h_authentication_failure_handling(abort):
    """A D2H record corrupted on its way to the host is zeroed in its host
    block and fails the batch (batch_end -1) -- or, with
    SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE=1, the reference's behaviour: the
    process aborts (secure_infer.cpp:2514-2524).  Host code only, under
    AddressSanitizer with the HIP stand-in."""
    exe = build("address")
    env = {**os.environ, "ASAN_OPTIONS": "halt_on_error=1:detect_leaks=0"}
    if abort:
        env["SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE"] = "1"
    r = subprocess.run([str(exe), "d2h_failure"], capture_output=True, text=True, timeout=300, env=env)
    report = r.stdout + r.stderr
    assert "AddressSanitizer" not in report, report[-4000:]
    if abort:
        assert r.returncode in (-6, 134), report[-4000:]
        assert "aborting (SECURE_INFER_D2H_ABORT_ON_AUTH_FAILURE)" in r.stderr
        assert "D2H_FAILURE_REPORTED" not in r.stdout
    else:
        assert r.returncode == 0 and "D2H_FAILURE_REPORTED" in r.stdout, report[-4000:]
