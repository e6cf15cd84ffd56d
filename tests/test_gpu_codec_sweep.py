"""GPU parity sweep of the int8 / int4 transport codec over KV shapes: one to
eight heads, head dims 64 and 128 (odd head counts give column counts that
are not powers of two), reload and writeback.

Reload: packets from the oracle's encoder (the restatement of
transport_codec.py:22-42), sealed by OpenSSL, verified / decrypted /
dequantised on the device and compared with the oracle's decode
(optimized_decode.py:5-26), one tampered V record zeroed.  Writeback: KV
blocks quantised and sealed on the device, compared with OpenSSL over the
oracle's packets of the same blocks.  Bit-exact throughout.  The reference's
own decode_into output at 1, 4 and 8 heads (tests/golden/codec_decode_vectors.npz)
is reloaded through the device as well.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import oracle as O
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEY = bytes(range(0x70, 0x80))
SALT = b"\x13\x57\x9b\xdf"
SHAPES = [(1, 64), (2, 64), (1, 128), (3, 128), (8, 64), (8, 128)]


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _caches(nslots, heads, dim, rng=None):
    if rng is None:
        k = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV)
        k.view(torch.uint8).fill_(0x3C)
        return k, k.clone()
    data = O.f32_to_bf16(rng.standard_normal((2, nslots, 128, heads, dim), dtype=np.float32))
    return _dev(data[0].view(np.int16)), _dev(data[1].view(np.int16)), data


@pytest.mark.parametrize("bits", [8, 4])
def test_codec_reload_shapes(bits):
    rng = np.random.default_rng(8100 + bits)
    ticket = 100
    for heads, dim in SHAPES:
        print(f"int{bits} reload {heads} x {dim}", flush=True)
        nb, nslots, layer = 3, 8, 5
        blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
        kinds = [0] * nb + [1] * nb
        packets = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
        n = packets[0].size
        assert n == si.codec_width(bits, heads, dim)
        wire = W.build_wire(KEY, SALT, packets, kinds, layer, list(range(2 * nb)), ticket)
        wire[(nb + 2) * W.stride(n) + int(rng.integers(0, n))] ^= 0x80  # V record 2
        slots_np = rng.permutation(nslots)[:nb].astype(np.int64)
        ck, cv = _caches(nslots, heads, dim)
        sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
        staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
        fail = torch.zeros(1, dtype=torch.int32, device=DEV)
        sess.reload_layer(_dev(wire), n, 2 * nb, nb, ck, cv, _dev(np.concatenate([slots_np, slots_np])),
                          ticket_base=ticket, codec_bits=bits, heads=heads, head_dim=dim, layer=layer,
                          staging=staging, fail_count=fail)
        ticket += 2 * nb
        kk, vv = _host(ck), _host(cv)
        assert int(_host(fail)[0]) == 1, (heads, dim)
        for i in range(nb):
            s = slots_np[i]
            assert np.array_equal(kk[s].view(np.uint16), O.codec_decode(packets[i], heads, dim, bits, 0)), \
                (heads, dim, "K", i)
            if i == 2:
                assert not vv[s].any(), (heads, dim)
            else:
                assert np.array_equal(vv[s].view(np.uint16),
                                      O.codec_decode(packets[nb + i], heads, dim, bits, 1)), (heads, dim, "V", i)
        untouched = np.setdiff1d(np.arange(nslots), slots_np)
        assert np.all(kk[untouched].view(np.uint8) == 0x3C) and np.all(vv[untouched].view(np.uint8) == 0x3C)


@pytest.mark.parametrize("bits", [8, 4])
def test_codec_writeback_shapes(bits):
    rng = np.random.default_rng(8200 + bits)
    ticket = 100
    for heads, dim in SHAPES:
        print(f"int{bits} writeback {heads} x {dim}", flush=True)
        nb, nslots, layer = 3, 8, 9
        ck, cv, data = _caches(nslots, heads, dim, rng)
        slots_np = rng.permutation(nslots)[:nb].astype(np.int64)
        kinds = [0] * nb + [1] * nb
        packets = [O.codec_encode(data[kinds[r]][slots_np[r % nb]], bits, kinds[r], layer)
                   for r in range(2 * nb)]
        n = packets[0].size
        wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(2 * nb)), ticket)
        sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
        staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
        dw = _dev(wire)
        sess.writeback_layer(dw, n, 2 * nb, nb, ck, cv, _dev(np.concatenate([slots_np, slots_np])),
                             ticket_base=ticket, codec_bits=bits, heads=heads, head_dim=dim,
                             layer=layer, staging=staging)
        ww = _host(dw)
        expect = W.build_wire(KEY, SALT, packets, kinds, layer, list(range(2 * nb)), ticket, direction=2)
        ticket += 2 * nb
        st, toff = W.stride(n), W.align32(n)
        for r in range(2 * nb):
            o = r * st
            assert np.array_equal(ww[o:o + n], expect[o:o + n]), (heads, dim, r, "ciphertext")
            assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16]), (heads, dim, r, "tag")


@pytest.mark.parametrize("heads", [1, 4, 8])
def test_reload_matches_reference_decode_fixture(heads):
    """The fixture's packets (int8 / int4, K and V) sealed with OpenSSL and
    reloaded into a paged cache: every slot equals decode_into's output."""
    z = np.load(Path(__file__).resolve().parent / "golden" / "codec_decode_vectors.npz", allow_pickle=False)
    pre = "" if heads == 1 else f"h{heads}_"
    dim, layer, nslots = 128, 3, 6
    for bits in (8, 4):
        print(f"int{bits} decode fixture {heads} heads", flush=True)
        packets = [z[f"{pre}packet_b{bits}_k0"], z[f"{pre}packet_b{bits}_k1"]]
        want = [z[f"{pre}decoded_b{bits}_k0"], z[f"{pre}decoded_b{bits}_k1"]]
        n = packets[0].size
        ticket = 500 + 10 * heads + bits
        wire = W.build_wire(KEY, SALT, packets, [0, 1], layer, [0, 0], ticket)
        ck, cv = _caches(nslots, heads, dim)
        sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
        staging = torch.zeros(2 * W.align32(n), dtype=torch.uint8, device=DEV)
        fail = torch.zeros(1, dtype=torch.int32, device=DEV)
        sess.reload_layer(_dev(wire), n, 2, 1, ck, cv, _dev(np.array([4, 4], np.int64)), ticket_base=ticket,
                          codec_bits=bits, heads=heads, head_dim=dim, layer=layer, staging=staging,
                          fail_count=fail)
        kk, vv = _host(ck), _host(cv)
        assert int(_host(fail)[0]) == 0
        assert np.array_equal(kk[4].view(np.uint16), want[0]), (heads, bits, "K")
        assert np.array_equal(vv[4].view(np.uint16), want[1]), (heads, bits, "V")
