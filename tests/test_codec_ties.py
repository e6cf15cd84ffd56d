"""Encoder parity at the quantiser's hard cases, against packets made by the
reference's own torch op sequence (tests/golden/codec_tie_vectors.npz, written
by tests/golden/make_codec_tie_vectors.py from transport_codec.py:24-36):
exact k + 0.5 ties, quotients a reciprocal-multiply would round wrongly,
constant groups and negative ranges.

* CPU: both oracle encoders (C and NumPy restatements) reproduce every packet
  byte, and the fixture really holds thousands of each hard case;
* GPU: the writeback quantiser (quant_kernel + AES-GCM seal), decrypted with
  OpenSSL, reproduces every packet byte.

tests/golden/codec_nonfinite_vectors.npz (same script) holds blocks with NaN,
+-inf and overflowing groups next to finite ones, where int4 K bytes pair
nibbles of two different groups: torch packs q[2i] + 16 q[2i+1] in float
before the uint8 cast, so a NaN quotient zeroes its partner
(transport_codec.py:33-34).  Every quantised byte and header byte must match;
parameter floats must match bit for bit where finite and be NaN where the
fixture's are (NaN payloads are not pinned)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

FIX = Path(__file__).resolve().parent / "golden" / "codec_tie_vectors.npz"
FIX_NONFINITE = Path(__file__).resolve().parent / "golden" / "codec_nonfinite_vectors.npz"
KEY = bytes(range(200, 216))
SALT = b"\x71\x72\x73\x74"


def fixture():
    z = np.load(FIX, allow_pickle=False)
    widths = z["widths"]
    rows = {int(w): z[f"packets_w{int(w)}"] for w in sorted(set(widths.tolist()))}
    seen = {w: 0 for w in rows}
    out = []
    for i in range(len(widths)):
        w = int(widths[i])
        out.append((z["blocks"][i], int(z["bits"][i]), int(z["kinds"][i]), rows[w][seen[w]]))
        seen[w] += 1
    return out, int(z["layer"]), z["ties"], z["recip_differs"]


def nonfinite_fixture():
    z = np.load(FIX_NONFINITE, allow_pickle=False)
    return [(z["blocks"][i], int(z["bits"][i]), int(z["kinds"][i]), z[f"packet_{i}"])
            for i in range(len(z["bits"]))], int(z["layer"])


def packet_mismatch(got: np.ndarray, want: np.ndarray, bits: int, heads: int, dim: int) -> str:
    """'' if got equals want: quantised bytes and header exactly, parameter
    floats bit for bit unless the expected one is NaN (then got must be NaN)."""
    qb = 128 * heads * dim * bits // 8
    sb = 2 * heads * dim * 4
    if got.size != want.size:
        return f"width {got.size} != {want.size}"
    bad = np.flatnonzero(got[:qb] != want[:qb])
    if bad.size:
        return f"{bad.size} quantised bytes differ, first at {bad[:5]}"
    pw = want[qb:qb + 2 * sb].view(np.float32)
    pg = got[qb:qb + 2 * sb].view(np.float32)
    nan = np.isnan(pw)
    if not np.array_equal(np.isnan(pg), nan):
        return "NaN parameters differ"
    if not np.array_equal(pg[~nan].view(np.uint32), pw[~nan].view(np.uint32)):
        return "finite parameters differ"
    if not np.array_equal(got[qb + 2 * sb:], want[qb + 2 * sb:]):
        return "header differs"
    return ""


def test_nonfinite_fixture_pairs_nan_with_finite_nibbles():
    """The fixture really exercises the pairing: int4 K holds bytes where
    exactly one of the two elements has a NaN quotient (so the byte is 0
    although its other nibble would not be)."""
    import torch
    cases, _ = nonfinite_fixture()
    assert {(b, k) for _, b, k, _ in cases} == {(8, 0), (8, 1), (4, 0), (4, 1)}
    blk = next(c[0] for c in cases if c[1] == 4 and c[2] == 0)
    x = torch.from_numpy(blk.view(np.int16).copy()).view(torch.bfloat16).float()
    g = x.reshape(2, 64, *x.shape[1:])
    lo, hi = g.amin(1, keepdim=True), g.amax(1, keepdim=True)
    q = ((g - lo) / ((hi - lo) / 15).clamp_min(1e-12)).round().clamp(0, 15).reshape(-1).numpy()
    a, b = q[0::2], q[1::2]
    one_nan = np.isnan(a) ^ np.isnan(b)
    partner = np.where(np.isnan(a), b, a)
    assert int((one_nan & (partner > 0)).sum()) > 100


@pytest.mark.parametrize("encoder", ["c", "numpy"])
def test_oracle_encoders_match_torch_on_nonfinite_groups(encoder):
    cases, layer = nonfinite_fixture()
    enc = O.codec_encode if encoder == "c" else O.np_codec_encode
    for blk, bits, kind, want in cases:
        msg = packet_mismatch(enc(blk, bits, kind, layer), want, bits, blk.shape[1], blk.shape[2])
        assert not msg, f"bits {bits} kind {kind}: {msg}"


def test_fixture_holds_the_hard_cases():
    cases, _, ties, recip = fixture()
    assert len(cases) == 8
    assert {(b, k) for _, b, k, _ in cases} == {(8, 0), (8, 1), (4, 0), (4, 1)}
    assert ties.min() > 1000 and recip.min() > 1000


@pytest.mark.parametrize("encoder", ["c", "numpy"])
def test_oracle_encoders_match_torch_at_ties(encoder):
    cases, layer, _, _ = fixture()
    enc = O.codec_encode if encoder == "c" else O.np_codec_encode
    for blk, bits, kind, want in cases:
        got = enc(blk, bits, kind, layer)
        assert got.size == want.size
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"bits {bits} kind {kind}: {bad.size} bytes differ, first at {bad[:5]}"


def gpu_writeback_packets(sel, layer, bits):
    """Packets of the GPU writeback quantiser + seal for the fixture cases
    `sel` (K blocks then V blocks), each decrypted and authenticated with
    OpenSSL; returns [(packet, expected)] in record order."""
    import torch

    import secure_infer_amd as si
    from tests import wire as W
    ks = [c for c in sel if c[2] == 0]
    vs = [c for c in sel if c[2] == 1]
    heads, dim = sel[0][0].shape[1], sel[0][0].shape[2]
    nb = len(ks)
    assert nb == len(vs)
    nslots = 5
    slot_ids = np.array([3, 0], np.int64)[:nb]
    ck = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device="cuda")
    cv = torch.zeros_like(ck)
    for i in range(nb):
        ck[int(slot_ids[i])] = torch.from_numpy(ks[i][0].view(np.int16)).cuda()
        cv[int(slot_ids[i])] = torch.from_numpy(vs[i][0].view(np.int16)).cuda()
    n = si.codec_width(bits, heads, dim)
    kinds = [0] * nb + [1] * nb
    t0 = 31000 + bits
    wire = torch.from_numpy(W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nb)) * 2, t0)).cuda()
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device="cuda")
    sess.writeback_layer(wire, n, 2 * nb, nb, ck, cv, torch.from_numpy(np.concatenate([slot_ids, slot_ids])).cuda(),
                         ticket_base=t0, codec_bits=bits, heads=heads, head_dim=dim, layer=layer, staging=staging)
    torch.cuda.synchronize()
    ww = wire.cpu().numpy().reshape(2 * nb, W.stride(n))
    toff = W.align32(n)
    out = []
    for r, want in enumerate([c[3] for c in ks] + [c[3] for c in vs]):
        ok, pt = O.ossl_gcm_decrypt(KEY, O.iv12_from_words(W.record_iv(SALT, t0 + r)),
                                    ww[r, toff + 32:toff + 96].tobytes(), ww[r, :n], ww[r, toff:toff + 16].tobytes())
        assert ok, f"record {r} failed authentication"
        out.append((np.asarray(pt), want))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_gpu_quantiser_matches_torch_at_ties(bits):
    cases, layer, _, _ = fixture()
    sel = [c for c in cases if c[1] == bits]
    for r, (pt, want) in enumerate(gpu_writeback_packets(sel, layer, bits)):
        bad = np.flatnonzero(pt != want)
        assert bad.size == 0, f"record {r}: {bad.size} bytes differ, first at {bad[:5]}"


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_gpu_quantiser_matches_torch_on_nonfinite_groups(bits):
    cases, layer = nonfinite_fixture()
    sel = [c for c in cases if c[1] == bits]
    heads, dim = sel[0][0].shape[1], sel[0][0].shape[2]
    for r, (pt, want) in enumerate(gpu_writeback_packets(sel, layer, bits)):
        msg = packet_mismatch(pt, want, bits, heads, dim)
        assert not msg, f"bits {bits} record {r}: {msg}"
