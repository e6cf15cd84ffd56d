"""The C-ABI library loads and exports every symbol include/*.h declares
(no compute calls: these run without a GPU)."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))
LIB = ROOT / "secure_infer_amd" / "_lib" / "libsecure_infer.so"


def declared_functions():
    names = []
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if name.startswith("secure_infer_") and name not in names:
                names.append(name)
    return names


def test_header_declares_reference_entry_points():
    names = declared_functions()
    for must in ("secure_infer_gpu_gcm_decrypt_verify_aad_do", "secure_infer_gpu_gcm_encrypt_tag_do",
                 "secure_infer_gpu_reload_layer", "secure_infer_gpu_writeback_layer",
                 "secure_infer_recovery_wait_layer_authentication",
                 "secure_infer_register_host_range_ex", "secure_infer_h2d_layer_group_begin"):
        assert must in names


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "build libsecure_infer.so first (python -m secure_infer_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_python_binding_covers_header():
    from secure_infer_amd import _lib
    assert set(declared_functions()) == set(_lib.SIGNATURES)
    lib = _lib.load()
    for name in _lib.SIGNATURES:
        assert hasattr(lib, name)


def test_host_only_entry_points_run_without_gpu():
    import secure_infer_amd as si
    assert si.wire_stride(262144) == 262144 + 96
    assert si.wire_stride(31) == 32 + 96
    assert si.codec_width(8, 8, 128) == 147472
    assert si.codec_width(4, 4, 128) == 40976
    t1, t2 = si.new_transfer_ticket(), si.new_transfer_ticket()
    assert t2 == t1 + 1 and t1 >= 1
    assert si.replay_reserve(10 ** 12 + t1) and not si.replay_reserve(10 ** 12 + t1)


def test_host_iv_and_aad_match_oracle():
    import numpy as np
    import torch
    import secure_infer_amd as si
    from oracle import oracle as O
    base = bytes.fromhex("deadbeef") + bytes(12)
    for ticket, off, nonce in ((1, 0, 0), (2 ** 40 + 3, 7, 5)):
        assert si.derive_transfer_iv(base, ticket, off, nonce) == O.derive_transfer_iv(base, ticket, off, nonce)
    pool = torch.zeros((6, 128, 2, 64), dtype=torch.bfloat16)
    si.clear_host_ranges()
    si.register_host_range(pool, layer_id=9, tensor_kind=1)
    blk = pool[4]
    aad = si.build_gcm_aad(blk.data_ptr(), blk.numel() * 2, 1, 123)
    assert aad == O.build_gcm_aad(1, 1, 9, 4, 0, blk.numel() * 2, 123)
    # unregistered address: deterministic descriptor keyed by the address
    other = np.zeros(64, np.uint8)
    aad2 = si.build_gcm_aad(other.ctypes.data, 64, 2, 5)
    assert aad2[5] == 2 and aad2[8:12] == b"\xff\xff\xff\xff"
    si.clear_host_ranges()
    with pytest.raises(ValueError):
        si.build_gcm_aad(blk.data_ptr(), 16, 3, 1)


def test_registering_a_range_again_relabels_it():
    """secure_infer.cpp:1066-1091: the same [base, base + bytes) registered
    again takes the new layer, kind and block size (no stale duplicate);
    the two-argument form (:1093-1097) registers layer and kind unknown."""
    import ctypes as ct
    import torch
    import secure_infer_amd as si
    from oracle import oracle as O
    from secure_infer_amd import _lib
    pool = torch.zeros((6, 128, 2, 64), dtype=torch.bfloat16)
    blk = pool[4]
    nbytes = blk.numel() * 2
    si.clear_host_ranges()
    try:
        si.register_host_range(pool, layer_id=9, tensor_kind=1)
        si.register_host_range(pool, layer_id=3, tensor_kind=0)
        assert si.build_gcm_aad(blk.data_ptr(), nbytes, 1, 77) == O.build_gcm_aad(1, 0, 3, 4, 0, nbytes, 77)
        si.clear_host_ranges()
        _lib.load().secure_infer_register_host_range(ct.c_void_p(pool.data_ptr()), pool.numel() * 2)
        aad = si.build_gcm_aad(blk.data_ptr(), nbytes, 2, 78)
        # no block size: the block id is the byte offset into the range
        assert aad == O.build_gcm_aad(2, 0xFF, 0xFFFFFFFF, 4 * nbytes, 0, nbytes, 78)
    finally:
        si.clear_host_ranges()


def test_error_returns_before_any_device_work():
    """The reference's error contract (0 / -1, launcher.asc returns -1 on null or
    zero arguments): invalid calls are rejected on the host, so they run here
    without a GPU."""
    import ctypes as ct

    from secure_infer_amd import _lib
    L = _lib.load()
    v = ct.c_void_p
    one = v(1)
    # kernel mirrors: null pointers / zero sizes
    assert L.secure_infer_gpu_gcm_decrypt_verify_aad_do(None, None, one, one, one, one, one, 16,
                                                        0, 0, 0, 2, None, 0) == -1
    assert L.secure_infer_gpu_gcm_decrypt_verify_aad_do(None, one, one, one, one, one, one, 0,
                                                        0, 0, 0, 2, None, 0) == -1
    assert L.secure_infer_gpu_gcm_decrypt_verify_aad_do(None, one, one, one, one, one, one, 16,
                                                        0, 0, 0, 2, None, 64) == -1  # AAD length, no AAD
    assert L.secure_infer_gpu_gcm_encrypt_tag_do(None, None, one, one, one, one, 16, 0, 0, 0, 2,
                                                 None, 0) == -1
    # sessions and layer entry points
    out = v()
    assert L.secure_infer_gpu_session_create(None, None, 0, 1024, ct.byref(out)) == -1
    assert L.secure_infer_gpu_reload_layer(None, None, None) == -1
    assert L.secure_infer_gpu_writeback_layer(None, None, None) == -1
    desc = _lib.SiReloadDesc(nrec=0)
    assert L.secure_infer_gpu_reload_layer(None, None, ct.byref(desc)) == -1
    assert L.secure_infer_h2d_swap(None, None, one, 16, 1, one, 16, 1, one, 0, 0, 0, 0, 0, 0, None) == -1
    # D2H brackets without a batch (secure_infer.cpp:2707-2970 semantics)
    assert L.secure_infer_d2h_group_begin(1) == -1
    assert L.secure_infer_d2h_group_end() == 0
    assert L.secure_infer_d2h_batch_device_barrier() == -1
    assert L.secure_infer_d2h_batch_end() == 0
    assert L.secure_infer_d2h_swap(None, None, one, 16, 1, one, 16, 1, one, 1, 0, 0, 0, 0, 0) == -1
    # layer groups nest (secure_infer.cpp:5883-5903) and are thread-local
    assert L.secure_infer_h2d_layer_group_begin(4) == 0
    assert L.secure_infer_h2d_layer_group_begin(4) == 0
    assert L.secure_infer_h2d_layer_group_end() == 0
    assert L.secure_infer_h2d_layer_group_end() == 0
    assert L.secure_infer_h2d_layer_group_end() == -1
    errors = []

    def other_thread():
        errors.append(L.secure_infer_h2d_layer_group_end())  # no group on this thread
    import threading
    assert L.secure_infer_h2d_layer_group_begin(2) == 0
    t = threading.Thread(target=other_thread)
    t.start()
    t.join()
    assert errors == [-1]
    assert L.secure_infer_h2d_layer_group_end() == 0
    # layer prefetch (a bf16 block of 1 head x 64 is 16,384 B): each call breaks
    # one argument -- null pools / mapping / group table, no groups, an empty
    # group, a host block outside the pool, a bad codec -- and is refused
    # before the (stand-in) session is touched
    m = (ct.c_int64 * 4)(0, 0, 1, 1)
    starts, rows, zero = (ct.c_uint32 * 1)(0), (ct.c_uint32 * 1)(2), (ct.c_uint32 * 1)(0)
    sess, bb = v(1), 16384
    assert L.secure_infer_h2d_prefetch_layer(sess, None, one, bb, 2, m, starts, rows, 1, 0, 0, 1, 64) == -1
    assert L.secure_infer_h2d_prefetch_layer(sess, one, one, bb, 2, None, starts, rows, 1, 0, 0, 1, 64) == -1
    assert L.secure_infer_h2d_prefetch_layer(sess, one, one, bb, 2, m, None, rows, 1, 0, 0, 1, 64) == -1
    assert L.secure_infer_h2d_prefetch_layer(sess, one, one, bb, 2, m, starts, rows, 0, 0, 0, 1, 64) == -1
    assert L.secure_infer_h2d_prefetch_layer(sess, one, one, bb, 2, m, starts, zero, 1, 0, 0, 1, 64) == -1
    assert L.secure_infer_h2d_prefetch_layer(sess, one, one, bb, 1, m, starts, rows, 1, 0, 0, 1, 64) == -1
    assert L.secure_infer_h2d_prefetch_layer(sess, one, one, bb, 2, m, starts, rows, 1, 0, 3, 1, 64) == -1
    # kernel clock: null / zero arguments, nothing clocked since arming
    words = ct.c_uint64()
    assert L.secure_infer_gpu_clock_next_layers(None, 16, 1) == -1
    assert L.secure_infer_gpu_clock_next_layers(one, 0, 1) == -1
    assert L.secure_infer_gpu_clock_next_layers(one, 16, 0) == -1
    assert L.secure_infer_gpu_clock_next_layers(one, 1 << 62, 8) == -1          # words overflow
    assert L.secure_infer_gpu_clock_next_layers(one, 16, 2) == 0
    assert L.secure_infer_gpu_clock_layers_used(ct.byref(words), 1) == -1      # no layer call yet
    assert L.secure_infer_gpu_clock_layers_used(ct.byref(words), 0) == -1
    assert L.secure_infer_gpu_clock_rate_khz(None) == -1
    # tracking and tuning
    assert L.secure_infer_recovery_track_layer(0, None, one) == -1
    assert L.secure_infer_gpu_set_chunk_rows(0) == -1
    assert L.secure_infer_gpu_set_chunk_rows(257) == -1
    assert L.secure_infer_gpu_set_chunk_rows(8) == 0
    assert L.secure_infer_gpu_set_chunk_rows(3) == 0
    assert L.secure_infer_gpu_set_straddle_rows(-1) == -1
    assert L.secure_infer_gpu_set_straddle_rows(257) == -1
    assert L.secure_infer_gpu_set_straddle_rows(6) == 0
    # IV / AAD builders
    iv = (ct.c_uint8 * 16)()
    assert L.secure_infer_derive_transfer_iv(iv, 0, 0, 0, iv) == -1          # ticket 0 is reserved
    aad = (ct.c_uint8 * 64)()
    assert L.secure_infer_build_gcm_aad(one, 16, 3, 1, 0, 0, aad) == 0      # direction must be 1 or 2
    assert L.secure_infer_build_gcm_aad(one, 16, 1, 0, 0, 0, aad) == 0      # ticket 0


def test_swaps_refuse_ids_outside_their_pools():
    """secure_infer_h2d_swap checks every (host block, device slot) of its
    mapping against the pool sizes before it touches the session, a ring or
    the device: an id outside [0, host_nblocks) or [0, nslots) refuses the
    whole call.  (The session pointer below is never dereferenced: the
    refusal comes first.)"""
    import ctypes as ct

    import numpy as np

    from secure_infer_amd import _lib
    L = _lib.load()
    host = np.zeros(4 * 256, np.uint8)
    fake_session = ct.c_void_p(16)
    dev = ct.c_void_p(4096)

    def h2d(mapping, nhost=4, nslots=8):
        m = np.ascontiguousarray(np.array(mapping, np.int64).reshape(-1, 2))
        return L.secure_infer_h2d_swap(None, fake_session, host.ctypes.data_as(ct.c_void_p), 256, nhost, dev,
                                       256, nslots, m.ctypes.data_as(ct.c_void_p), m.shape[0], 0, 0, 0, 0, 0,
                                       None)
    assert h2d([[4, 0]]) == -1            # host block == host_nblocks
    assert h2d([[0, 1], [-1, 2]]) == -1   # negative host block
    assert h2d([[0, 8]]) == -1            # slot == nslots
    assert h2d([[1, 0], [2, -3]]) == -1   # negative slot
    assert h2d([[0, 0]], nhost=0) == -1   # empty host pool
    assert h2d([[0, 0]], nslots=0) == -1  # empty cache


def test_replay_set_rejects_reused_tickets():
    import secure_infer_amd as si
    base = 7 * 10 ** 15
    assert si.replay_reserve(base + 5)
    assert si.replay_reserve(base + 7)
    assert si.replay_reserve(base + 6)      # fills the gap between two runs
    for t in (base + 5, base + 6, base + 7):
        assert not si.replay_reserve(t)
    assert si.replay_reserve(base + 4) and si.replay_reserve(base + 8)
    assert not si.replay_reserve(base + 4)
    assert si.replay_reserve(0)             # ticket 0 is never recorded (secure_infer.cpp:779)
    assert si.replay_reserve(0)


def test_prefetch_retirement_is_a_no_op():
    """EncodedStore binds secure_infer_retire_transfer_prefetches
    unconditionally (transport_codec.py:50); this library has no speculative
    pools, so both calls return without effect."""
    import ctypes as ct
    from secure_infer_amd import _lib
    lib = ct.CDLL(str(_lib.LIB_PATH))
    lib.secure_infer_retire_transfer_prefetches()
    lib.secure_infer_invalidate_transfer_prefetches()
