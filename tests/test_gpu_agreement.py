"""The session key agreement's device code (si_agree.hip) and an agreed
session end to end (secure_infer_gpu_session_agree; the reference's device
session, secure_infer.cpp:447-521, key_agreement.aicpu:9-49):

* device X25519 equals RFC 7748's vectors and the oracle restatement
  (itself pinned to the RFC and to OpenSSL) on random scalars and
  u-coordinates, including u with its top bit set and u >= p;
* device keyed BLAKE2b equals hashlib over keys of 0-64 bytes, messages
  around the 128-byte block boundary and digest sizes 4-64;
* the kernels' context built on the device from a key equals the host
  builder's image byte for byte;
* an agreed session reloads host-sealed records (the host's copy of the key)
  through the device's own context bit-exactly and writes back records the
  host authenticates; two agreements yield different hash subkeys;
* a wrong device proof or a low-order host public value makes no session.
"""
import ctypes as ct
import hashlib
import os

import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import agreement as A
from secure_infer_amd import _lib
from tests import wire as W
from tests.test_agreement import RFC_5_2

pytestmark = pytest.mark.gpu
DEV = "cuda"


def dev_x25519(k: bytes, u: bytes) -> bytes:
    out = ct.create_string_buffer(32)
    assert _lib.load().secure_infer_test_x25519(k, u, out) == 0
    return out.raw


def dev_blake2b(key: bytes, msg: bytes, n: int) -> bytes:
    out = ct.create_string_buffer(n)
    assert _lib.load().secure_infer_test_blake2b(key or None, len(key), msg or None, len(msg), out, n) == 0
    return out.raw


def test_device_x25519():
    for k, u, want in RFC_5_2:
        assert dev_x25519(bytes.fromhex(k), bytes.fromhex(u)).hex() == want
    rng = np.random.default_rng(171)
    p = 2 ** 255 - 19
    cases = [(rng.bytes(32), rng.bytes(32)) for _ in range(6)]
    cases.append((rng.bytes(32), (p + 5).to_bytes(32, "little")))           # u >= p
    cases.append((rng.bytes(32), bytes(31) + b"\x80"))                     # only the ignored top bit
    cases.append((rng.bytes(32), (9).to_bytes(32, "little")))              # the base point
    for k, u in cases:
        assert dev_x25519(k, u) == A.x25519(k, u)


def test_device_blake2b():
    rng = np.random.default_rng(172)
    for klen in (0, 16, 32, 64):
        for mlen in (0, 1, 127, 128, 129, 256, 1000):
            key, msg = rng.bytes(klen), rng.bytes(mlen)
            for n in (4, 16, 32, 64):
                assert dev_blake2b(key, msg, n) == hashlib.blake2b(msg, key=key, digest_size=n).digest()


@pytest.mark.parametrize("max_record_bytes", [4096, 262144, 147472])
def test_device_context_equals_host_context(max_record_bytes):
    L = _lib.load()
    key = os.urandom(16)
    n = L.secure_infer_test_context_image(key, max_record_bytes, 0, None, 0)
    assert n > 0
    host_img = ct.create_string_buffer(n)
    dev_img = ct.create_string_buffer(n)
    assert L.secure_infer_test_context_image(key, max_record_bytes, 0, host_img, n) == n
    assert L.secure_infer_test_context_image(key, max_record_bytes, 1, dev_img, n) == n
    a = np.frombuffer(host_img.raw, np.uint8)
    b = np.frombuffer(dev_img.raw, np.uint8)
    assert np.array_equal(a, b), f"first difference at byte {int(np.argmax(a != b))}"


def test_agreed_session_end_to_end():
    rng = np.random.default_rng(173)
    heads, dim, ncpu, nslots = 2, 128, 8, 16
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession.agree(session_nonce=11, max_record_bytes=shape.record_bytes)
    other = si.GcmSession.agree(session_nonce=11, max_record_bytes=shape.record_bytes)
    assert sess.key is None and sess.iv_salt is None
    assert sess.hash_subkey != other.hash_subkey  # fresh keys per agreement
    si.clear_host_ranges()
    try:
        hk = torch.from_numpy(np.stack(W.bf16_blocks(rng, ncpu, heads, dim)).view(np.int16)).contiguous()
        hv = torch.from_numpy(np.stack(W.bf16_blocks(rng, ncpu, heads, dim)).view(np.int16)).contiguous()
        si.register_host_range(hk, 0, 0)
        si.register_host_range(hv, 0, 1)
        ck = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV)
        cv = torch.zeros_like(ck)
        m = torch.tensor([[7, 3], [0, 12], [5, 1]], dtype=torch.int64)
        nt = si.NativeTransfer(sess, shape)
        nt.single_layer_kv_transfer(((hk, hv), m), (ck, cv))
        assert nt.wait_layer(0) == 0
        for c, s in m.tolist():
            assert torch.equal(ck[s].cpu(), hk[c]) and torch.equal(cv[s].cpu(), hv[c])
        # and back: sealed on the device, authenticated by the host
        bk, bv = torch.zeros_like(hk), torch.zeros_like(hv)
        back = torch.stack([m[:, 1], m[:, 0]], 1).contiguous()
        si.D2HTransfer(sess, shape).store([(ck, cv)], [(bk, bv)], back)
        for c, _ in m.tolist():
            assert torch.equal(bk[c], hk[c]) and torch.equal(bv[c], hv[c])
    finally:
        si.clear_host_ranges()
        sess.close()
        other.close()


@pytest.mark.parametrize("mode", [1, 2], ids=["bad_proof", "low_order_point"])
def test_agreement_refuses_a_bad_proof_or_a_low_order_point(mode):
    """The host rejects a device proof that does not match its own key
    derivation (secure_infer.cpp:487-499), and the device refuses an all-zero
    shared secret (a low-order host public value, key_agreement.aicpu:33-35);
    either way no session is made.  The fault is one shot."""
    L = _lib.load()
    assert L.secure_infer_test_tamper_agree(mode) == 0
    try:
        with pytest.raises(RuntimeError, match="session_agree"):
            si.GcmSession.agree(max_record_bytes=4096)
    finally:
        L.secure_infer_test_tamper_agree(0)
    si.GcmSession.agree(max_record_bytes=4096).close()
