"""GPU edge cases of the layer entry points: out-of-range slot ids, K-only /
V-only layers, record sizes that are not whole blocks, explicit IV words with
a 32-bit counter wrap, every record tampered, codec parameter tampering,
NaN and infinities in the KV of the codec paths.
All comparisons are bit-exact against OpenSSL / the oracle."""
import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import oracle as O
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEY = bytes(range(0x50, 0x60))
SALT = b"\x0a\x0b\x0c\x0d"
FILL = 0x3C


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def statuses(wire: np.ndarray, n: int, nrec: int) -> np.ndarray:
    st, toff = W.stride(n), W.align32(n)
    return np.array([int.from_bytes(wire[r * st + toff + 16:r * st + toff + 20].tobytes(), "little")
                     for r in range(nrec)])


def byte_caches(nslots, n):
    k = torch.full((nslots, n), FILL, dtype=torch.uint8, device=DEV)
    return k, torch.full_like(k, FILL)


def test_reload_bad_slots_fail_closed():
    rng = np.random.default_rng(201)
    n, nb, nslots = 8192, 3, 6
    pl = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(2 * nb)]
    kinds = [0] * nb + [1] * nb
    wire = W.build_wire(KEY, SALT, pl, kinds, 1, list(range(2 * nb)), 300)
    slots = np.array([2, -1, 5, nslots, 0, 4], np.int64)  # records 1 and 3 out of range
    ck, cv = byte_caches(nslots, n)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = dev(wire)
    sess.reload_layer(dw, n, 2 * nb, nb, ck, cv, dev(slots), ticket_base=300, fail_count=fail)
    kk, vv, ww = host(ck), host(cv), host(dw)
    assert int(host(fail)[0]) == 2
    assert list(statuses(ww, n, 2 * nb)) == [1, 0, 1, 0, 1, 1]
    assert np.array_equal(kk[2], pl[0]) and np.array_equal(kk[5], pl[2])
    assert np.array_equal(vv[0], pl[4]) and np.array_equal(vv[4], pl[5])
    for s in (0, 1, 3, 4):
        assert (kk[s] == FILL).all()
    for s in (1, 2, 3, 5):
        assert (vv[s] == FILL).all()


@pytest.mark.parametrize("n_k", [0, 4])
def test_reload_single_kind_layers(n_k):
    rng = np.random.default_rng(211 + n_k)
    n, nrec, nslots = 16384, 4, 8
    pl = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(nrec)]
    kinds = [0 if r < n_k else 1 for r in range(nrec)]
    wire = W.build_wire(KEY, SALT, pl, kinds, 2, list(range(nrec)), 400)
    slots = rng.permutation(nslots)[:nrec].astype(np.int64)
    ck, cv = byte_caches(nslots, n)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    sess.reload_layer(dev(wire), n, nrec, n_k, ck, cv, dev(slots), ticket_base=400)
    got, other = (host(ck), host(cv)) if n_k else (host(cv), host(ck))
    for r in range(nrec):
        assert np.array_equal(got[slots[r]], pl[r])
    assert (other == FILL).all()


@pytest.mark.parametrize("n", [4000, 4001, 65535])
def test_reload_partial_last_block(n):
    rng = np.random.default_rng(221 + n)
    nb, nslots = 2, 5
    pl = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(2 * nb)]
    kinds = [0] * nb + [1] * nb
    wire = W.build_wire(KEY, SALT, pl, kinds, 0, list(range(2 * nb)), 500)
    wire[W.stride(n) * 3 + n - 1] ^= 0x01  # V record 1: last (partial-block) byte
    slots = np.array([1, 3, 0, 4], np.int64)
    slot_bytes = (n + 15) // 16 * 16 + 32
    ck, cv = byte_caches(nslots, slot_bytes)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    sess.reload_layer(dev(wire), n, 2 * nb, nb, ck, cv, dev(slots), ticket_base=500, fail_count=fail)
    kk, vv = host(ck), host(cv)
    assert int(host(fail)[0]) == 1
    assert np.array_equal(kk[1][:n], pl[0]) and np.array_equal(kk[3][:n], pl[1])
    assert np.array_equal(vv[0][:n], pl[2])
    assert not vv[4][:n].any()                        # failed record zeroed
    assert (kk[1][n:] == FILL).all() and (vv[4][n:] == FILL).all()  # nothing past the record


def test_reload_explicit_iv_words_counter_wrap():
    rng = np.random.default_rng(231)
    n, nrec, nslots = 4096, 3, 4
    key = KEY
    h = O.hash_subkey(key)
    ivs = [(0x01020304, 0x05060708, 0x090a0b0c, 0xFFFFFFF8),  # wraps after 8 blocks
           (0xdeadbeef, 0, 1, 2),
           (0x11111111, 0x22222222, 0x33333333, 0x7FFFFFFF)]
    pl = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(nrec)]
    st, toff = W.stride(n), W.align32(n)
    wire = np.zeros(nrec * st, np.uint8)
    for r in range(nrec):
        aad = rng.integers(0, 256, 64, dtype=np.uint8)
        c, tag = O.gcm_encrypt_tag(key, h, ivs[r], aad, pl[r])
        wire[r * st:r * st + n] = c
        wire[r * st + toff:r * st + toff + 16] = np.frombuffer(tag, np.uint8)
        wire[r * st + toff + 32:r * st + toff + 96] = aad
    words = dev(np.array(ivs, np.uint32).reshape(-1))
    ck, cv = byte_caches(nslots, n)
    sess = si.GcmSession(key, SALT, 0, max_record_bytes=n)
    dw = dev(wire)
    sess.reload_layer(dw, n, nrec, nrec, ck, cv, dev(np.array([3, 0, 2], np.int64)), iv_words_dev=words)
    kk, ww = host(ck), host(dw)
    assert list(statuses(ww, n, nrec)) == [1, 1, 1]
    for r, s in enumerate([3, 0, 2]):
        assert np.array_equal(kk[s], pl[r]), f"record {r}"


def test_reload_every_record_tampered():
    rng = np.random.default_rng(241)
    n, nb, nslots = 32768, 4, 8
    pl = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(2 * nb)]
    kinds = [0] * nb + [1] * nb
    wire = W.build_wire(KEY, SALT, pl, kinds, 3, list(range(2 * nb)), 600)
    for r in range(2 * nb):
        wire[r * W.stride(n) + W.align32(n) + (r % 16)] ^= 0xFF  # every tag
    slots = rng.permutation(nslots)[:nb].astype(np.int64)
    ck, cv = byte_caches(nslots, n)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = dev(wire)
    sess.reload_layer(dw, n, 2 * nb, nb, ck, cv, dev(np.concatenate([slots, slots])), ticket_base=600,
                      fail_count=fail)
    kk, vv, ww = host(ck), host(cv), host(dw)
    assert int(host(fail)[0]) == 2 * nb
    assert not statuses(ww, n, 2 * nb).any()
    for s in slots:
        assert not kk[s].any() and not vv[s].any()


def test_writeback_bad_slot_reported():
    rng = np.random.default_rng(251)
    heads, dim, nslots, layer = 2, 128, 6, 4
    data = O.f32_to_bf16(rng.standard_normal((2, nslots, 128, heads, dim), dtype=np.float32))
    ck, cv = dev(data[0].view(np.int16)), dev(data[1].view(np.int16))
    slots = np.array([5, nslots + 3, 1, 0], np.int64)  # K record 1 out of range
    nb = 2
    kinds = [0, 0, 1, 1]
    n = 128 * heads * dim * 2
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, [0, 1, 0, 1], 700)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = dev(wire)
    sess.writeback_layer(dw, n, 4, nb, ck, cv, dev(slots), ticket_base=700, layer=layer, fail_count=fail)
    ww = host(dw)
    assert int(host(fail)[0]) == 1
    plain = [data[0][5], None, data[1][1], data[1][0]]
    expect = W.build_wire(KEY, SALT, [p.view(np.uint8).reshape(-1) if p is not None else np.zeros(n, np.uint8)
                                      for p in plain], kinds, layer, [0, 1, 0, 1], 700, direction=2)
    st, toff = W.stride(n), W.align32(n)
    for r in (0, 2, 3):
        o = r * st
        assert np.array_equal(ww[o:o + n], expect[o:o + n])
        assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16])


@pytest.mark.parametrize("where", ["scale", "low", "header"])
def test_codec_reload_parameter_tamper(where):
    rng = np.random.default_rng(261)
    heads, dim, bits, layer, nb, nslots = 2, 128, 8, 1, 2, 4
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    kinds = [0] * nb + [1] * nb
    packets = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
    n = packets[0].size
    qb, sb, _ = O.codec_sizes(bits, heads, dim)
    off = {"scale": qb + 5, "low": qb + sb + 7, "header": qb + 2 * sb + 4}[where]
    wire = W.build_wire(KEY, SALT, packets, kinds, layer, list(range(2 * nb)), 800)
    wire[2 * W.stride(n) + off] ^= 0x10  # V record 0
    slots = np.array([3, 1], np.int64)
    ck = torch.full((nslots, 128, heads, dim), 0x3C3C, dtype=torch.int16, device=DEV)
    cv = torch.full_like(ck, 0x3C3C)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    sess.reload_layer(dev(wire), n, 2 * nb, nb, ck, cv, dev(np.concatenate([slots, slots])), ticket_base=800,
                      codec_bits=bits, heads=heads, head_dim=dim, layer=layer, staging=staging,
                      fail_count=fail)
    kk, vv = host(ck), host(cv)
    assert int(host(fail)[0]) == 1
    assert not vv[3].any()
    assert np.array_equal(vv[1].view(np.uint16), O.codec_decode(packets[3], heads, dim, bits, 1))
    for i, s in enumerate(slots):
        assert np.array_equal(kk[s].view(np.uint16), O.codec_decode(packets[i], heads, dim, bits, 0))


def nonfinite_block(rng, heads, dim):
    """bf16 block with NaN and +-inf in a few K groups / V rows."""
    x = rng.standard_normal((128, heads, dim), dtype=np.float32)
    x[5, 0, 3] = np.nan
    x[70, 1, 9] = np.inf
    x[20, 1, 100], x[30, 1, 100] = np.inf, -np.inf
    x[99, 0, 64] = -np.inf
    return O.f32_to_bf16(x)


def params_match(a, b):
    """float32 parameters equal bit for bit, NaN payloads aside."""
    fa, fb = a.view(np.float32), b.view(np.float32)
    na, nb_ = np.isnan(fa), np.isnan(fb)
    return bool(np.array_equal(na, nb_) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb_]))


@pytest.mark.parametrize("bits", [8, 4])
def test_codec_nonfinite_kv(bits):
    # NaN / inf in the KV: the quantisers propagate NaN through the group's
    # min / max like x.amin / x.amax, the dequantiser turns NaN results into
    # bf16 0x7fc0.  Writeback packets (staging) against the oracle, their
    # ciphertext checked by the oracle's GCM decrypt; reload of the oracle's
    # packets bit-exact against the oracle's decode.
    rng = np.random.default_rng(77 + bits)
    heads, dim, nb, nslots, layer = 2, 128, 2, 6, 4
    data = np.stack([np.stack([nonfinite_block(rng, heads, dim) for _ in range(nslots)]) for _ in range(2)])
    ck, cv = dev(data[0].view(np.int16)), dev(data[1].view(np.int16))
    slots_np = np.array([4, 1], np.int64)
    kinds = [0] * nb + [1] * nb
    expect = [O.codec_encode(data[kinds[r]][slots_np[r % nb]], bits, kinds[r], layer) for r in range(2 * nb)]
    n = expect[0].size
    qb, sb, _ = O.codec_sizes(bits, heads, dim)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    ticket0 = 700
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(2 * nb)), ticket0)
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
    dw = dev(wire)
    slots2 = dev(np.concatenate([slots_np, slots_np]))
    sess.writeback_layer(dw, n, 2 * nb, nb, ck, cv, slots2, ticket_base=ticket0, codec_bits=bits,
                         heads=heads, head_dim=dim, layer=layer, staging=staging)
    st_h, ww = host(staging), host(dw)
    h = O.hash_subkey(KEY)
    st, toff = W.stride(n), W.align32(n)
    for r in range(2 * nb):
        pkt = st_h[r * toff:r * toff + n]
        assert np.array_equal(pkt[:qb], expect[r][:qb]), f"record {r} q"
        assert params_match(pkt[qb:qb + 2 * sb], expect[r][qb:qb + 2 * sb]), f"record {r} params"
        assert np.array_equal(pkt[qb + 2 * sb:], expect[r][qb + 2 * sb:]), f"record {r} header"
        o = r * st
        status, plain = O.gcm_decrypt_verify(KEY, h, W.record_iv(SALT, ticket0 + r), ww[o + toff + 32:o + toff + 96],
                                             ww[o:o + n], ww[o + toff:o + toff + 16].tobytes())
        assert status == 1 and np.array_equal(plain, pkt), f"record {r} ciphertext / tag"
    # reload of the oracle's packets
    wire2 = W.build_wire(KEY, SALT, expect, kinds, layer, list(range(2 * nb)), ticket0 + 10)
    ck2 = torch.zeros_like(ck)
    cv2 = torch.zeros_like(cv)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    stage2 = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
    sess.reload_layer(dev(wire2), n, 2 * nb, nb, ck2, cv2, slots2, ticket_base=ticket0 + 10, codec_bits=bits,
                      heads=heads, head_dim=dim, layer=layer, staging=stage2, fail_count=fail)
    kk, vv = host(ck2).view(np.uint16), host(cv2).view(np.uint16)
    assert int(host(fail)[0]) == 0
    for i in range(nb):
        s = slots_np[i]
        assert np.array_equal(kk[s], O.codec_decode(expect[i], heads, dim, bits, 0)), f"K slot {s}"
        assert np.array_equal(vv[s], O.codec_decode(expect[nb + i], heads, dim, bits, 1)), f"V slot {s}"
        assert (kk[s] == 0x7FC0).any() and (vv[s] == 0x7FC0).any()
