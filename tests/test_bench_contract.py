"""bench.py's host-side contract, without a GPU: it refuses more than one
GPU before touching one, its workloads' algorithmic bytes are the figures the
roofline divides by, the tickets, IV words and AADs it builds its wire records
with equal the library's own (so the device verifies what the bench seals),
its ledger parser reads the library's H2D ledger rows, and its ROCTx ranges do
nothing where the ROCTx library is absent."""
import importlib.util
import subprocess
import sys
from pathlib import Path
from unittest import mock

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and not r.stdout


def test_algorithmic_bytes_per_layer():
    """Per record, reload: ciphertext read + bf16 write + tag + AAD + status;
    writeback: bf16 read + ciphertext write + tag + AAD.  The four workloads
    the baseline table derives its roofline targets from, byte for byte."""
    import secure_infer_amd as si
    b = load_bench()
    want = {"reload_bf16_llama3_8b_6144tok": 50_339_712, "reload_int8_llama3_8b_8192tok": 52_441_600,
            "reload_int4_qwen2_5_7b_8192tok": 22_032_896, "writeback_int4_llama3_70b_32768tok": 176_209_920}
    for name, total in want.items():
        c = b.CONFIGS[name]
        block = 128 * c["heads"] * c["dim"] * 2
        nbytes = block if c["bits"] == 0 else si.codec_width(c["bits"], c["heads"], c["dim"])
        assert 2 * c["blocks"] * b.algorithmic_bytes_per_record(c["op"], nbytes, block) == total, name
    assert b.DEFAULT in b.CONFIGS and b.CONFIGS[b.DEFAULT]["op"] == "reload"


def test_tickets_iv_words_and_aads_match_the_library():
    import secure_infer_amd as si
    from secure_infer_amd.gcm import reference_ticket_order
    b = load_bench()
    # reload: the reference's submission order (16-block groups from the tail, K then V)
    nb = 41
    t = b.record_tickets("reload", nb, 100)
    for i, (kind, blk) in enumerate(reference_ticket_order(nb, b.LOAD_CHUNK_BLOCKS)):
        assert t[kind * nb + blk] == 100 + i
    assert sorted(t.tolist()) == list(range(100, 100 + 2 * nb))
    # writeback: K blocks then V blocks
    assert b.record_tickets("writeback", 5, 7).tolist() == list(range(7, 17))
    # IV words: salt || BE64(nonce + ticket) || BE32(2), as the library derives them
    salt = bytes.fromhex("a1b2c3d4")
    tickets = np.array([5, 2 ** 40 + 9], np.int64)
    w = b.iv_words_of(salt, 3, tickets)
    for i, tk in enumerate(tickets.tolist()):
        iv = si.derive_transfer_iv(salt + bytes(12), tk, 0, 3)
        assert b"".join(int(x).to_bytes(4, "big") for x in w[i]) == iv
    # AAD of a registered host block
    pool = torch.zeros((6, 128, 2, 64), dtype=torch.bfloat16)
    si.clear_host_ranges()
    try:
        si.register_host_range(pool, layer_id=9, tensor_kind=1)
        blk = pool[4]
        nbytes = blk.numel() * 2
        assert b.aad_bytes(1, 1, 9, 4, nbytes, 123) == si.build_gcm_aad(blk.data_ptr(), nbytes, 1, 123)
        assert b.aad_bytes(2, 1, 9, 4, nbytes, 124) == si.build_gcm_aad(blk.data_ptr(), nbytes, 2, 124)
    finally:
        si.clear_host_ranges()


def test_ledger_split_reads_the_ledger_rows(tmp_path):
    b = load_bench()
    csv = tmp_path / "h2d.csv"
    csv.write_text("layer,kind,records,record_bytes,source,seal_us,h2d_copy_us,kernel_us\n"
                   "0,2,32,1024,prefetched,10,20,5\n"
                   "0,2,32,1024,prefetched,30,40,7\n"
                   "1,2,32,1024,sealed,100,50,6\n")
    out = b.ledger_split(csv, 1)
    assert out["prefetched"]["launches"] == 2 and out["prefetched"]["launches_per_layer"] == 2.0
    assert out["prefetched"]["seal_us_per_layer"] == 40.0 and out["prefetched"]["kernel_us_per_layer"] == 12.0
    assert out["sealed"]["h2d_copy_us_per_layer"] == 50.0
    assert b.ledger_split(tmp_path / "absent.csv", 1) == {}


def test_roctx_ranges_are_no_ops_without_the_library():
    b = load_bench()
    b.Range._fns = None
    with mock.patch("ctypes.CDLL", side_effect=OSError("absent")):
        with b.Range("timed:x"):
            pass
    assert b.Range._fns == ()
    b.Range._fns = None
