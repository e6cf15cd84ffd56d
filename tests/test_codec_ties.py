"""Encoder parity at the quantiser's hard cases, against packets made by the
reference's own torch op sequence (tests/golden/codec_tie_vectors.npz, written
by tests/golden/make_codec_tie_vectors.py from transport_codec.py:24-36):
exact k + 0.5 ties, quotients a reciprocal-multiply would round wrongly,
constant groups and negative ranges.

* CPU: both oracle encoders (C and NumPy restatements) reproduce every packet
  byte, and the fixture really holds thousands of each hard case;
* GPU: the writeback quantiser (quant_kernel + AES-GCM seal), decrypted with
  OpenSSL, reproduces every packet byte."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

FIX = Path(__file__).resolve().parent / "golden" / "codec_tie_vectors.npz"
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


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_gpu_quantiser_matches_torch_at_ties(bits):
    import torch

    import secure_infer_amd as si
    from tests import wire as W
    cases, layer, _, _ = fixture()
    sel = [c for c in cases if c[1] == bits]
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
    for r, want in enumerate([c[3] for c in ks] + [c[3] for c in vs]):
        ok, pt = O.ossl_gcm_decrypt(KEY, O.iv12_from_words(W.record_iv(SALT, t0 + r)),
                                    ww[r, toff + 32:toff + 96].tobytes(), ww[r, :n], ww[r, toff:toff + 16].tobytes())
        assert ok, f"record {r} failed authentication"
        bad = np.flatnonzero(pt != want)
        assert bad.size == 0, f"record {r}: {bad.size} bytes differ, first at {bad[:5]}"
