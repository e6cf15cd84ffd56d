"""GPU tests of the kernel-level entry points that complete the reference's
AICPU launcher set (launcher.asc): GHASH with its three flags, the AAD-less
verify launchers, the verify-xor and keystream batches, and the device half
of the key agreement.  Each is checked against OpenSSL and the oracle (its
GHASH, CTR keystream and X25519 / BLAKE2b exchange) on the same inputs,
bit-exactly, including failing tags and unaligned buffers.
"""
import os
import struct

import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import agreement as A
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(bytes(a), np.uint8).copy()).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def record(rng, n, aad_bytes):
    key, iv12 = rng.bytes(16), rng.bytes(12)
    aad, pt = rng.bytes(aad_bytes), rng.bytes(n)
    ct_, tag = O.ossl_gcm_encrypt(key, iv12, aad, pt)
    iv = struct.unpack(">III", iv12) + (2,)
    return key, iv, aad, np.frombuffer(pt, np.uint8), ct_, tag


def unaligned(a, off) -> torch.Tensor:
    """A device copy of `a` starting `off` bytes into a larger buffer."""
    a = np.frombuffer(bytes(a), np.uint8)
    big = torch.zeros(a.size + off + 3, dtype=torch.uint8, device=DEV)
    big[off:off + a.size] = torch.from_numpy(a.copy()).to(DEV)
    return big[off:off + a.size]


@pytest.mark.parametrize("aad_bytes", [64, 0, 20])
@pytest.mark.parametrize("n", [16, 31, 1000, 40976, 262144])
def test_ghash_flags_against_openssl_and_the_oracle(n, aad_bytes):
    rng = np.random.default_rng(n * 131 + aad_bytes)
    key, iv, aad, pt, ct_, tag = record(rng, n, aad_bytes)
    h = O.hash_subkey(key)
    ks = O.keystream(key, iv, n)
    mask = O.keystream(key, iv[:3] + (1,), 16)  # E_K(J0)
    dct, dh = unaligned(ct_, 1), dev(h)
    da = dev(aad) if aad_bytes else None
    out = torch.zeros(16, dtype=torch.uint8, device=DEV)
    # No flags: the GHASH value itself.
    si.ghash(dct, dh, out, aad=da)
    assert host(out).tobytes() == O.ghash(h, aad, ct_)
    # FINALIZE: the GCM tag.
    st = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    si.ghash(dct, dh, out, aad=da, tag_mask=dev(mask), status_out=st, flags=si.GHASH_FINALIZE_TAG)
    assert host(out).tobytes() == tag and int(host(st)[0]) == 1
    # FINALIZE | VERIFY | XOR: the authenticated release.
    plain = unaligned(np.zeros(n, np.uint8), 3)
    flags = si.GHASH_FINALIZE_TAG | si.GHASH_VERIFY_TAG | si.GHASH_XOR_ON_SUCCESS
    si.ghash(dct, dh, out, aad=da, tag_mask=dev(mask), expected_tag=dev(tag), keystream=dev(ks),
             plaintext_out=plain, status_out=st, flags=flags)
    assert int(host(st)[0]) == 1 and np.array_equal(host(plain), pt)
    # A wrong expected tag: status 0, the release zeroed, the computed tag still out.
    bad = bytearray(tag)
    bad[15] ^= 0x40
    plain2 = torch.full((n,), 0x5A, dtype=torch.uint8, device=DEV)
    si.ghash(dct, dh, out, aad=da, tag_mask=dev(mask), expected_tag=dev(bad), keystream=dev(ks),
             plaintext_out=plain2, status_out=st, flags=flags)
    assert int(host(st)[0]) == 0 and not host(plain2).any() and host(out).tobytes() == tag


def test_ghash_refuses_missing_flag_operands():
    dct, dh = dev(bytes(32)), dev(bytes(16))
    out = torch.zeros(16, dtype=torch.uint8, device=DEV)
    for flags in (si.GHASH_FINALIZE_TAG, si.GHASH_VERIFY_TAG, si.GHASH_XOR_ON_SUCCESS):
        with pytest.raises(RuntimeError):
            si.ghash(dct, dh, out, flags=flags)


@pytest.mark.parametrize("n", [16, 31, 4099, 262144])
def test_aad_less_verify_launchers(n):
    rng = np.random.default_rng(n + 7)
    key, iv, _, pt, ct_, tag = record(rng, n, 0)
    dk, dh, dct = dev(key), dev(O.hash_subkey(key)), dev(ct_)
    ks = torch.empty_like(dct)
    si.keystream(dk, ks, iv)
    for t, want in ((tag, 1), (bytes([tag[0] ^ 1]) + tag[1:], 0)):
        out = torch.full((n,), 0x77, dtype=torch.uint8, device=DEV)
        st, st2 = (torch.full((1,), 9, dtype=torch.int32, device=DEV) for _ in range(2))
        si.gcm_verify_xor(dct, dk, dh, dev(t), ks, out, st, iv)
        si.gcm_verify_only(dct, dk, dh, dev(t), st2, iv)
        assert int(host(st)[0]) == want and int(host(st2)[0]) == want
        assert np.array_equal(host(out), pt if want else np.zeros(n, np.uint8))


@pytest.mark.parametrize("aad_bytes", [64, 0])
def test_verify_xor_batch_and_keystream_batch(aad_bytes):
    rng = np.random.default_rng(29 + aad_bytes)
    n, count = 40976, 4
    key = rng.bytes(16)
    dk, dh = dev(key), dev(O.hash_subkey(key))
    ivs, aads, pts, cts, tags = [], [], [], [], []
    for r in range(count):
        iv12 = rng.bytes(12)
        ivs.append(struct.unpack(">III", iv12) + (2,))
        aads.append(rng.bytes(aad_bytes))
        pts.append(np.frombuffer(rng.bytes(n), np.uint8))
        c, t = O.ossl_gcm_encrypt(key, iv12, aads[-1], pts[-1])
        cts.append(c)
        tags.append(bytearray(t))
    tags[2][5] ^= 1  # record 2 fails
    kss = [torch.empty(n, dtype=torch.uint8, device=DEV) for _ in range(count)]
    si.keystream_batch(dk, kss, ivs)
    for r in range(count):
        assert np.array_equal(host(kss[r]), O.keystream(key, ivs[r], n))
    outs = [torch.full((n,), 0x33, dtype=torch.uint8, device=DEV) for _ in range(count)]
    sts = [torch.full((1,), 9, dtype=torch.int32, device=DEV) for _ in range(count)]
    si.gcm_verify_xor_batch(dk, dh, [dev(c) for c in cts], [dev(t) for t in tags], kss, outs, sts, ivs,
                            aads=[dev(a) for a in aads] if aad_bytes else None)
    for r in range(count):
        ok = r != 2
        assert int(host(sts[r])[0]) == int(ok)
        assert np.array_equal(host(outs[r]), pts[r] if ok else np.zeros(n, np.uint8))
    with pytest.raises(RuntimeError):  # more than four records
        si.gcm_verify_xor_batch(dk, dh, [dev(cts[0])] * 5, [dev(tags[0])] * 5, kss + kss[:1], outs + outs[:1],
                                sts + sts[:1], ivs + ivs[:1])


def test_key_agreement_launcher_matches_the_host_half():
    host_secret, challenge = os.urandom(32), os.urandom(32)
    host_public = A.public_key(host_secret)
    dkey = torch.zeros(16, dtype=torch.uint8, device=DEV)
    dpub = torch.zeros(32, dtype=torch.uint8, device=DEV)
    proof = torch.zeros(32, dtype=torch.uint8, device=DEV)
    status = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    si.key_agreement(dev(host_public), dev(challenge), dkey, dpub, proof, status)
    assert int(host(status)[0]) == 0
    key, expected, _ = A.host_half(host_secret, host(dpub).tobytes(), challenge)
    assert host(proof).tobytes() == expected and host(dkey).tobytes() == key
    # A second run draws a fresh device secret.
    dpub2 = torch.zeros_like(dpub)
    si.key_agreement(dev(host_public), dev(challenge), dkey, dpub2, proof, status)
    assert int(host(status)[0]) == 0 and host(dpub2).tobytes() != host(dpub).tobytes()
    # The all-zero (low-order) host public value: the shared secret is zero.
    si.key_agreement(dev(bytes(32)), dev(challenge), dkey, dpub, proof, status)
    assert int(host(status)[0]) == 2
