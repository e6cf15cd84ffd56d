"""GPU parity tests: the HIP path through the C-ABI against the oracle and
OpenSSL (the reference's host AES-128-GCM) on the same key, IV and inputs.

Integer / byte work: every comparison is bit-exact.  Ported from the
reference's device known-answer test (tests/crypto_smoke.py: sizes 16, 31,
32768, 262144 B, 64-B AAD; device encrypt == host AES-GCM, host encrypt ->
device decrypt, keystream + verify_xor) plus fail-closed tamper cases.
"""
import struct

import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import oracle as O
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rand_bytes(rng, n):
    return rng.integers(0, 256, n, dtype=np.uint8)


SIZES = [16, 31, 1000, 32768, 40976, 147472, 262144]


@pytest.mark.parametrize("n", SIZES)
def test_kernel_mirrors_match_openssl(n):
    rng = np.random.default_rng(n)
    key, iv12, aad = rand_bytes(rng, 16), rand_bytes(rng, 12), rand_bytes(rng, 64)
    pt = rand_bytes(rng, n)
    ref_ct, ref_tag = O.ossl_gcm_encrypt(key.tobytes(), iv12.tobytes(), aad, pt)
    h = np.frombuffer(O.hash_subkey(key.tobytes()), np.uint8)
    iv = struct.unpack(">III", iv12.tobytes()) + (2,)
    dk, dh, da, dp = dev(key), dev(h), dev(aad), dev(pt)
    c = torch.empty_like(dp)
    tag = torch.zeros(16, dtype=torch.uint8, device=DEV)
    si.gcm_encrypt_tag(dp, dk, dh, c, tag, iv, aad=da)
    assert np.array_equal(host(c), ref_ct), "device encryption mismatch"
    assert host(tag).tobytes() == ref_tag

    dc, dt = dev(ref_ct), dev(np.frombuffer(ref_tag, np.uint8))
    out = torch.zeros_like(dc)
    st = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    si.gcm_decrypt_verify(dc, dk, dh, dt, out, st, iv, aad=da)
    assert int(host(st)[0]) == 1 and np.array_equal(host(out), pt)

    ks = torch.empty_like(dc)
    si.keystream(dk, ks, iv)
    assert np.array_equal(host(ks), O.keystream(key.tobytes(), iv, n))
    out2 = torch.zeros_like(dc)
    st2 = torch.zeros(1, dtype=torch.int32, device=DEV)
    si.gcm_verify_xor(dc, dk, dh, dt, ks, out2, st2, iv, aad=da)
    assert int(host(st2)[0]) == 1 and np.array_equal(host(out2), pt)

    st3 = torch.zeros(1, dtype=torch.int32, device=DEV)
    si.gcm_verify_only(dc, dk, dh, dt, st3, iv, aad=da)
    assert int(host(st3)[0]) == 1

    back = torch.empty_like(dc)
    si.aes_ctr(dc, dk, back, iv)
    assert np.array_equal(host(back), pt)


def test_no_aad_and_unaligned_buffers():
    rng = np.random.default_rng(5)
    n = 4099
    key, pt = rand_bytes(rng, 16), rand_bytes(rng, n)
    iv = (0x11223344, 0x55667788, 0x99AABBCC, 2)
    ref_ct, ref_tag = O.ossl_gcm_encrypt(key.tobytes(), O.iv12_from_words(iv), b"", pt)
    h = np.frombuffer(O.hash_subkey(key.tobytes()), np.uint8)
    dk, dh = dev(key), dev(h)
    big = torch.zeros(n + 3, dtype=torch.uint8, device=DEV)
    big[1:n + 1] = dev(pt)
    cbig = torch.zeros(n + 5, dtype=torch.uint8, device=DEV)
    tag = torch.zeros(16, dtype=torch.uint8, device=DEV)
    si.gcm_encrypt_tag(big[1:n + 1], dk, dh, cbig[3:n + 3], tag, iv, nbytes=n)
    assert np.array_equal(host(cbig)[3:n + 3], ref_ct) and host(tag).tobytes() == ref_tag
    out = torch.zeros(n + 7, dtype=torch.uint8, device=DEV)
    st = torch.zeros(1, dtype=torch.int32, device=DEV)
    si.gcm_decrypt_verify(cbig[3:n + 3], dk, dh, tag, out[5:n + 5], st, iv, nbytes=n)
    o = host(out)
    assert int(host(st)[0]) == 1 and np.array_equal(o[5:n + 5], pt)
    assert not o[:5].any() and not o[n + 5:].any()


@pytest.mark.parametrize("where", ["ct_first", "ct_last", "tag", "aad"])
def test_tampered_record_fails_closed(where):
    rng = np.random.default_rng(11)
    n = 262144
    key, aad, pt = rand_bytes(rng, 16), rand_bytes(rng, 64), rand_bytes(rng, n)
    iv = (0xA1B2C3D4, 0, 77, 2)
    ct_, tag = O.ossl_gcm_encrypt(key.tobytes(), O.iv12_from_words(iv), aad, pt)
    tag = bytearray(tag)
    if where == "ct_first":
        ct_[0] ^= 1
    elif where == "ct_last":
        ct_[-1] ^= 0x80
    elif where == "tag":
        tag[15] ^= 4
    else:
        aad = aad.copy()
        aad[63] ^= 2
    h = np.frombuffer(O.hash_subkey(key.tobytes()), np.uint8)
    out = torch.full((n,), 0x5A, dtype=torch.uint8, device=DEV)
    st = torch.full((1,), 9, dtype=torch.int32, device=DEV)
    si.gcm_decrypt_verify(dev(ct_), dev(key), dev(h), dev(np.frombuffer(bytes(tag), np.uint8)), out, st,
                          iv, aad=dev(aad))
    assert int(host(st)[0]) == 0
    assert not host(out).any()
    ref_st, _ = O.gcm_decrypt_verify(key.tobytes(), h.tobytes(), iv, aad, ct_, bytes(tag))
    assert ref_st == 0


def test_auth_gate():
    data = torch.full((1000,), 3, dtype=torch.uint8, device=DEV)
    ok = torch.ones(1, dtype=torch.int32, device=DEV)
    si.auth_gate(data, ok)
    assert host(data).min() == 3
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    si.auth_gate(data, bad)
    assert not host(data).any()


# ---------------------------------------------------------------- layer level

KEY = bytes(range(100, 116))
SALT = bytes.fromhex("c0ffee01")


def make_caches(nslots, heads, dim, fill=0x3C):
    k = torch.full((nslots, 128, heads, dim), 0, dtype=torch.int16, device=DEV)
    v = torch.full((nslots, 128, heads, dim), 0, dtype=torch.int16, device=DEV)
    k.view(torch.uint8).fill_(fill)
    v.view(torch.uint8).fill_(fill)
    return k, v


@pytest.mark.parametrize("chunk_rows,straddle", [(16, 10), (1, 10), (3, 6), (3, 0), (16, 0), (64, 0)])
def test_reload_layer_bf16(chunk_rows, straddle):
    rng = np.random.default_rng(21)
    heads, dim, nb, nslots, layer = 8, 128, 6, 32, 4
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    payloads = [b.view(np.uint8).reshape(-1) for b in blocks]
    kinds = [0] * nb + [1] * nb
    cpu_ids = list(rng.permutation(100)[:nb]) * 2
    ticket0 = 1000
    wire = W.build_wire(KEY, SALT, payloads, kinds, layer, cpu_ids, ticket0)
    wire[3 * W.stride(payloads[0].size) + 100] ^= 0x20  # record 3 (a K block) tampered
    slots_np = rng.permutation(nslots)[:nb].astype(np.int64)
    slots = dev(np.concatenate([slots_np, slots_np]))
    ck, cv = make_caches(nslots, heads, dim)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=payloads[0].size)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    si.set_chunk_rows(chunk_rows)
    si.set_straddle_rows(straddle)
    try:
        dw = dev(wire)
        sess.reload_layer(dw, payloads[0].size, 2 * nb, nb, ck, cv, slots, ticket_base=ticket0,
                          fail_count=fail)
        kk, vv, ww = host(ck), host(cv), host(dw)
    finally:
        si.set_chunk_rows(si.gcm.DEFAULT_CHUNK_ROWS)
        si.set_straddle_rows(si.gcm.DEFAULT_STRADDLE_ROWS)
    st = W.stride(payloads[0].size)
    toff = W.align32(payloads[0].size)
    statuses = [int(ww[r * st + toff + 16:r * st + toff + 20].view(np.uint32)[0]) for r in range(2 * nb)]
    assert statuses == [1, 1, 1, 0, 1, 1] + [1] * nb
    assert int(host(fail)[0]) == 1
    used = set(slots_np.tolist())
    for i in range(nb):
        s = slots_np[i]
        if i == 3:
            assert not kk[s].any()
        else:
            assert np.array_equal(kk[s].view(np.uint16), blocks[i])
        assert np.array_equal(vv[s].view(np.uint16), blocks[nb + i])
    for s in range(nslots):
        if s not in used:
            assert np.all(kk[s].view(np.uint8) == 0x3C) and np.all(vv[s].view(np.uint8) == 0x3C)


@pytest.mark.parametrize("bits", [8, 4])
def test_reload_layer_codec(bits):
    rng = np.random.default_rng(31 + bits)
    heads, dim, nb, nslots, layer = 4, 128, 5, 16, 2
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    kinds = [0] * nb + [1] * nb
    packets = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
    n = packets[0].size
    assert n == si.codec_width(bits, heads, dim)
    ticket0 = 5000
    wire = W.build_wire(KEY, SALT, packets, kinds, layer, list(range(2 * nb)), ticket0)
    wire[(nb + 1) * W.stride(n) + n - 1] ^= 1  # V record 1: flip last ciphertext byte
    slots_np = rng.permutation(nslots)[:nb].astype(np.int64)
    ck, cv = make_caches(nslots, heads, dim)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    sess.reload_layer(dev(wire), n, 2 * nb, nb, ck, cv, dev(np.concatenate([slots_np, slots_np])),
                      ticket_base=ticket0, codec_bits=bits, heads=heads, head_dim=dim, layer=layer,
                      staging=staging, fail_count=fail)
    kk, vv = host(ck), host(cv)
    assert int(host(fail)[0]) == 1
    for i in range(nb):
        s = slots_np[i]
        assert np.array_equal(kk[s].view(np.uint16), O.codec_decode(packets[i], heads, dim, bits, 0))
        if i == 1:
            assert not vv[s].any()
        else:
            assert np.array_equal(vv[s].view(np.uint16),
                                  O.codec_decode(packets[nb + i], heads, dim, bits, 1))


@pytest.mark.parametrize("bits", [0, 8, 4])
def test_writeback_layer(bits):
    rng = np.random.default_rng(41 + bits)
    heads, dim, nb, nslots, layer = 8, 128, 4, 16, 7
    ck, cv = make_caches(nslots, heads, dim)
    data = O.f32_to_bf16(rng.standard_normal((2, nslots, 128, heads, dim), dtype=np.float32))
    ck.copy_(dev(data[0].view(np.int16)))
    cv.copy_(dev(data[1].view(np.int16)))
    slots_np = rng.permutation(nslots)[:nb].astype(np.int64)
    kinds = [0] * nb + [1] * nb
    if bits:
        plain = [O.codec_encode(data[kinds[r]][slots_np[r % nb]], bits, kinds[r], layer)
                 for r in range(2 * nb)]
    else:
        plain = [data[kinds[r]][slots_np[r % nb]].view(np.uint8).reshape(-1) for r in range(2 * nb)]
    n = plain[0].size
    ticket0 = 9000
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(2 * nb)), ticket0)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV) if bits else None
    dw = dev(wire)
    sess.writeback_layer(dw, n, 2 * nb, nb, ck, cv, dev(np.concatenate([slots_np, slots_np])),
                         ticket_base=ticket0, codec_bits=bits, heads=heads, head_dim=dim,
                         layer=layer, staging=staging)
    ww = host(dw)
    expect = W.build_wire(KEY, SALT, plain, kinds, layer, list(range(2 * nb)), ticket0, direction=2)
    st, toff = W.stride(n), W.align32(n)
    for r in range(2 * nb):
        o = r * st
        assert np.array_equal(ww[o:o + n], expect[o:o + n]), f"record {r} ciphertext"
        assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16]), f"record {r} tag"


@pytest.mark.parametrize("kinds_of", ["k_only", "v_only"])
def test_writeback_codec_one_kind(kinds_of):
    """The quantiser grid with K workgroups only or V workgroups only."""
    rng = np.random.default_rng(51 + len(kinds_of))
    heads, dim, nrec, nslots, layer, bits = 4, 128, 3, 8, 5, 4
    ck, cv = make_caches(nslots, heads, dim)
    data = O.f32_to_bf16(rng.standard_normal((2, nslots, 128, heads, dim), dtype=np.float32))
    ck.copy_(dev(data[0].view(np.int16)))
    cv.copy_(dev(data[1].view(np.int16)))
    slots_np = rng.permutation(nslots)[:nrec].astype(np.int64)
    n_k = nrec if kinds_of == "k_only" else 0
    kinds = [0 if r < n_k else 1 for r in range(nrec)]
    plain = [O.codec_encode(data[kinds[r]][slots_np[r]], bits, kinds[r], layer) for r in range(nrec)]
    n = plain[0].size
    ticket0 = 700
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nrec)), ticket0)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.zeros(nrec * W.align32(n), dtype=torch.uint8, device=DEV)
    dw = dev(wire)
    sess.writeback_layer(dw, n, nrec, n_k, ck, cv, dev(slots_np), ticket_base=ticket0, codec_bits=bits,
                         heads=heads, head_dim=dim, layer=layer, staging=staging)
    ww = host(dw)
    expect = W.build_wire(KEY, SALT, plain, kinds, layer, list(range(nrec)), ticket0, direction=2)
    st, toff = W.stride(n), W.align32(n)
    for r in range(nrec):
        o = r * st
        assert np.array_equal(ww[o:o + n], expect[o:o + n]), f"record {r} ciphertext"
        assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16]), f"record {r} tag"


@pytest.mark.parametrize("chunk_rows", [3, 16, 64])
def test_writeback_layer_straddling_shares(chunk_rows):
    """Encrypt with workgroup shares that straddle two records (straddle cost
    0, shares of at least chunk_rows rows), bf16 records of 65 rows."""
    rng = np.random.default_rng(61 + chunk_rows)
    heads, dim, nb, nslots, layer = 8, 128, 5, 16, 2
    ck, cv = make_caches(nslots, heads, dim)
    data = O.f32_to_bf16(rng.standard_normal((2, nslots, 128, heads, dim), dtype=np.float32))
    ck.copy_(dev(data[0].view(np.int16)))
    cv.copy_(dev(data[1].view(np.int16)))
    slots_np = rng.permutation(nslots)[:nb].astype(np.int64)
    kinds = [0] * nb + [1] * nb
    plain = [data[kinds[r]][slots_np[r % nb]].view(np.uint8).reshape(-1) for r in range(2 * nb)]
    n = plain[0].size
    ticket0 = 500
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(2 * nb)), ticket0)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    dw = dev(wire)
    si.set_chunk_rows(chunk_rows)
    si.set_straddle_rows(0)
    try:
        sess.writeback_layer(dw, n, 2 * nb, nb, ck, cv, dev(np.concatenate([slots_np, slots_np])),
                             ticket_base=ticket0, codec_bits=0, heads=heads, head_dim=dim, layer=layer)
        ww = host(dw)
    finally:
        si.set_chunk_rows(si.gcm.DEFAULT_CHUNK_ROWS)
        si.set_straddle_rows(si.gcm.DEFAULT_STRADDLE_ROWS)
    expect = W.build_wire(KEY, SALT, plain, kinds, layer, list(range(2 * nb)), ticket0, direction=2)
    st, toff = W.stride(n), W.align32(n)
    for r in range(2 * nb):
        o = r * st
        assert np.array_equal(ww[o:o + n], expect[o:o + n]), f"record {r} ciphertext"
        assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16]), f"record {r} tag"


@pytest.mark.parametrize("bits,extra", [(0, -1), (4, -1), (0, 0)])
def test_layer_pairs_of_whole_records(bits, extra):
    """More records than CUs (2 * CUs - 1 or 2 * CUs): the host lays out
    shares of two whole records (one placement table for both, segment 0's
    products parked in global memory), with an odd count a last share of one.
    Reload with tampered records at both positions of a pair and in the last
    share, then writeback parity against OpenSSL."""
    rng = np.random.default_rng(71 + bits - extra)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    heads, dim, layer = 1, 64, 3
    nrec = 2 * cus + extra
    nb = (nrec + 1) // 2
    nv = nrec - nb
    nslots = nb + 7
    kinds = [0] * nb + [1] * nv
    slots_np = np.concatenate([rng.permutation(nslots)[:nb], rng.permutation(nslots)[:nv]]).astype(np.int64)
    data = O.f32_to_bf16(rng.standard_normal((2, nslots, 128, heads, dim), dtype=np.float32))
    blocks = [data[kinds[r]][slots_np[r]] for r in range(nrec)]
    if bits:
        plain = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(nrec)]
    else:
        plain = [blocks[r].view(np.uint8).reshape(-1) for r in range(nrec)]
    n = plain[0].size
    st, toff = W.stride(n), W.align32(n)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.zeros(nrec * W.align32(n), dtype=torch.uint8, device=DEV) if bits else None

    # Writeback: device gather (+ quantise) + encrypt == OpenSSL.
    ck, cv = make_caches(nslots, heads, dim)
    ck.copy_(dev(data[0].view(np.int16)))
    cv.copy_(dev(data[1].view(np.int16)))
    ticket0 = 20000
    dw = dev(W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nrec)), ticket0))
    sess.writeback_layer(dw, n, nrec, nb, ck, cv, dev(slots_np), ticket_base=ticket0, codec_bits=bits,
                         heads=heads, head_dim=dim, layer=layer, staging=staging)
    ww = host(dw)
    expect = W.build_wire(KEY, SALT, plain, kinds, layer, list(range(nrec)), ticket0, direction=2)
    for r in range(nrec):
        o = r * st
        assert np.array_equal(ww[o:o + n], expect[o:o + n]), f"record {r} ciphertext"
        assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16]), f"record {r} tag"

    # Reload into fresh caches, records 0, 3 (both positions of a pair) and
    # the last (a share of its own) tampered.
    ticket1 = 30000
    wire = W.build_wire(KEY, SALT, plain, kinds, layer, list(range(nrec)), ticket1)
    bad = {0, 3, nrec - 1}
    for r in bad:
        wire[r * st + (r * 37) % n] ^= 0x10
    ck2, cv2 = make_caches(nslots, heads, dim)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = dev(wire)
    sess.reload_layer(dw, n, nrec, nb, ck2, cv2, dev(slots_np), ticket_base=ticket1, codec_bits=bits,
                      heads=heads, head_dim=dim, layer=layer, staging=staging, fail_count=fail)
    kk, vv, ww = host(ck2), host(cv2), host(dw)
    assert int(host(fail)[0]) == len(bad)
    for r in range(nrec):
        status = int(ww[r * st + toff + 16:r * st + toff + 20].view(np.uint32)[0])
        assert status == (0 if r in bad else 1), f"record {r} status"
        got = (kk if kinds[r] == 0 else vv)[slots_np[r]]
        if r in bad:
            assert not got.any(), f"record {r} not zeroed"
        elif bits:
            want = O.codec_decode(plain[r], heads, dim, bits, kinds[r])
            assert np.array_equal(got.view(np.uint16), want), f"record {r} decode"
        else:
            assert np.array_equal(got.view(np.uint16), blocks[r]), f"record {r} payload"


def test_native_transfer_wait_layer():
    rng = np.random.default_rng(51)
    heads, dim, nb, nslots = 2, 128, 3, 8
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=shape.record_bytes)
    ck, cv = make_caches(nslots, heads, dim)
    mapping = torch.tensor([[10, 5], [11, 2], [12, 7]], dtype=torch.int64)
    nt = si.NativeTransfer(sess, shape)
    tickets = []
    for layer in range(2):
        blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
        t0 = 20000 + 100 * layer
        wire = W.build_wire(KEY, SALT, [b.view(np.uint8).reshape(-1) for b in blocks],
                            [0] * nb + [1] * nb, layer, [10, 11, 12] * 2, t0)
        if layer == 1:
            wire[W.align32(shape.record_bytes)] ^= 1  # tag of record 0
        nt.single_layer_wire_transfer((dev(wire), mapping), (ck, cv), ticket_base=t0)
        tickets.append(blocks)
    assert nt.wait_layer(0) == 0
    assert nt.wait_layer(1) == -1
    kk = host(ck)
    assert not kk[5].any()  # layer 1 record 0 (K block -> slot 5) withheld
    assert np.array_equal(kk[2].view(np.uint16), tickets[1][1])


@pytest.mark.parametrize("bits", [0, 4])
def test_clocked_layer_launch(bits):
    """secure_infer_gpu_clock_next_layers: armed for two layer calls, every
    wave of each call's kernels (a reload, then a writeback) writes the device
    clock at its start and end into that call's words -- two words per wave,
    each start at or before its end, the reload's span positive and within
    the host's wall time -- the results are unchanged, and a third call is not
    clocked.  Stamps that do not fit leave the launch unstamped and are
    reported (-1), nothing is written past the words given, and the results
    are still right."""
    import ctypes as ct
    import time
    rng = np.random.default_rng(71 + bits)
    heads, dim, nb, nslots, layer, t0 = 4, 128, 6, 16, 3, 31000 + bits
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    kinds = [0] * nb + [1] * nb
    if bits:
        payloads = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
        want = np.stack([O.codec_decode(payloads[r], heads, dim, bits, kinds[r]) for r in range(2 * nb)])
    else:
        payloads = [blocks[r].view(np.uint8).reshape(-1) for r in range(2 * nb)]
        want = blocks
    n = payloads[0].size
    wire = dev(W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0))
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    ck, cv = make_caches(nslots, heads, dim)
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    slots = dev(np.concatenate([slot_ids, slot_ids]))
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV) if bits else None
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    wb = dev(W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nb)) * 2, t0 + 100))
    L = si._lib.load()
    khz = ct.c_uint64()
    assert L.secure_infer_gpu_clock_rate_khz(ct.byref(khz)) == 0 and khz.value > 0
    words = 1 << 15
    big = torch.iinfo(torch.int64).max
    stamps = torch.zeros(2 * words + 64, dtype=torch.int64, device=DEV)
    ptr = ct.c_void_p(stamps.data_ptr())

    def arm(nwords, layers):
        stamps[0::2] = big
        stamps[1::2] = 0
        assert L.secure_infer_gpu_clock_next_layers(ptr, nwords, layers) == 0

    def used(layers):
        u = (ct.c_uint64 * layers)()
        return L.secure_infer_gpu_clock_layers_used(u, layers), list(u)

    def reload():
        sess.reload_layer(wire, n, 2 * nb, nb, ck, cv, slots, ticket_base=t0, codec_bits=bits, heads=heads,
                          head_dim=dim, layer=layer, staging=staging, fail_count=fail)

    def writeback():
        sess.writeback_layer(wb, n, 2 * nb, nb, ck, cv, slots, ticket_base=t0 + 100, codec_bits=bits, heads=heads,
                             head_dim=dim, layer=layer, staging=staging)

    def check_reload():
        assert int(fail.item()) == 0
        idx = dev(slot_ids)
        assert torch.equal(ck.index_select(0, idx), dev(want[:nb].view(np.int16)))
        assert torch.equal(cv.index_select(0, idx), dev(want[nb:].view(np.int16)))

    assert L.secure_infer_gpu_clock_next_layers(None, 16, 1) == -1
    assert L.secure_infer_gpu_clock_next_layers(ptr, 0, 1) == -1
    assert L.secure_infer_gpu_clock_next_layers(ptr, 16, 0) == -1
    arm(words, 2)
    assert used(1)[0] == -1  # nothing clocked yet
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    reload()
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - w0) * 1e6
    check_reload()
    writeback()
    torch.cuda.synchronize()
    rc, u = used(2)
    assert rc == 0 and all(0 < x <= words and x % 2 == 0 for x in u)
    assert used(3)[0] == -1
    got = stamps.cpu().numpy()
    for l in range(2):
        seg = got[l * words:(l + 1) * words]
        st, en = seg[0:u[l]:2], seg[1:u[l]:2]
        assert (st != big).all() and (en != 0).all() and (st <= en).all()
        assert (seg[u[l]::2] == big).all() and (seg[u[l] + 1::2] == 0).all()  # nothing past its waves
    seg = got[:words]
    span_us = (seg[1:u[0]:2].max() - seg[0:u[0]:2].min()) * 1e3 / khz.value
    assert 0 < span_us <= wall_us
    expect = W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0 + 100, direction=2)
    g = host(wb).reshape(2 * nb, W.stride(n))
    ex = expect.reshape(2 * nb, W.stride(n))
    assert np.array_equal(g[:, :n], ex[:, :n])
    # the arming covered two calls: a third leaves the stamps alone
    before = stamps.clone()
    reload()
    torch.cuda.synchronize()
    assert torch.equal(stamps, before)
    # too few words: the kernels that do not fit stamp nothing; reported
    arm(2, 1)
    ck.zero_()
    cv.zero_()
    reload()
    torch.cuda.synchronize()
    assert used(1)[0] == -1
    assert (stamps[0::2] == big).all() and (stamps[1::2] == 0).all()
    check_reload()


@pytest.mark.parametrize("bits", [0, 4])
def test_timed_layer_launch(bits):
    """secure_infer_gpu_time_next_layer: the next layer call (reload, then
    writeback) launches its first and last kernels with the caller's events;
    the interval is positive and within the host's wall time around the call,
    the results are unchanged (bit-exact, statuses 1), and the arming is one
    shot (the following call leaves the events alone)."""
    import time
    rng = np.random.default_rng(61 + bits)
    heads, dim, nb, nslots, layer, t0 = 4, 128, 6, 16, 2, 30000 + bits
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    kinds = [0] * nb + [1] * nb
    if bits:
        payloads = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
        want = np.stack([O.codec_decode(payloads[r], heads, dim, bits, kinds[r]) for r in range(2 * nb)])
    else:
        payloads = [blocks[r].view(np.uint8).reshape(-1) for r in range(2 * nb)]
        want = blocks
    n = payloads[0].size
    wire = dev(W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0))
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    ck, cv = make_caches(nslots, heads, dim)
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    slots = dev(np.concatenate([slot_ids, slot_ids]))
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV) if bits else None
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    L = si._lib.load()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    b.record()
    torch.cuda.synchronize()
    assert L.secure_infer_gpu_time_next_layer(None, None) == -1
    assert L.secure_infer_gpu_time_next_layer(a.cuda_event, b.cuda_event) == 0
    w0 = time.perf_counter()
    sess.reload_layer(wire, n, 2 * nb, nb, ck, cv, slots, ticket_base=t0, codec_bits=bits, heads=heads,
                      head_dim=dim, layer=layer, staging=staging, fail_count=fail)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - w0) * 1e3
    ms = a.elapsed_time(b)
    assert 0 < ms <= wall_ms
    assert int(fail.item()) == 0
    idx = dev(slot_ids)
    assert torch.equal(ck.index_select(0, idx), dev(want[:nb].view(np.int16)))
    assert torch.equal(cv.index_select(0, idx), dev(want[nb:].view(np.int16)))
    # one shot: the next (unarmed) call does not move the events
    sess.reload_layer(wire, n, 2 * nb, nb, ck, cv, slots, ticket_base=t0, codec_bits=bits, heads=heads,
                      head_dim=dim, layer=layer, staging=staging, fail_count=fail)
    torch.cuda.synchronize()
    assert a.elapsed_time(b) == ms
    # writeback, timed the same way, seals what OpenSSL seals
    wb = dev(W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nb)) * 2, t0 + 100))
    assert L.secure_infer_gpu_time_next_layer(a.cuda_event, b.cuda_event) == 0
    sess.writeback_layer(wb, n, 2 * nb, nb, ck, cv, slots, ticket_base=t0 + 100, codec_bits=bits, heads=heads,
                         head_dim=dim, layer=layer, staging=staging)
    torch.cuda.synchronize()
    assert a.elapsed_time(b) > 0
    expect = W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0 + 100, direction=2)
    got = host(wb).reshape(2 * nb, W.stride(n))
    ex = expect.reshape(2 * nb, W.stride(n))
    toff = W.align32(n)
    assert np.array_equal(got[:, :n], ex[:, :n]) and np.array_equal(got[:, toff:toff + 16], ex[:, toff:toff + 16])
