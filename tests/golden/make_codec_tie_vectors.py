"""Writes tests/golden/codec_tie_vectors.npz: packets of the reference's
transport-codec encoder on crafted KV blocks, computed with torch on the CPU.

The encoder is the op sequence of transport_codec.encode
(secure_infer/kv_offload/transport_codec.py:24-36), restated here with the
same torch calls (its module cannot be imported: it imports vLLM), so the
fixture carries torch's own float semantics: amin / amax, the division by
(2^bits - 1), clamp_min(1e-12), the division by the scale, round-half-even,
clamp, nibble packing and the packet layout.  The blocks are crafted so that
the quantiser's hard cases occur many times:

* exact ties: (x - low) / scale == k + 0.5 exactly (scales 1, 2, 0.5, 0.25);
* quotients where a * RN(1/scale) rounds to another integer than a / scale
  (found by search in float32), i.e. a division formed as a multiply by the
  reciprocal would fail;
* all-equal groups (scale clamps to 1e-12), negative ranges, and random
  N(0, 1) columns.

Counts of each case are stored with the vectors; tests/test_codec_ties.py
asserts them and checks the oracle encoders (C and NumPy) and the GPU
quantiser against the packets.

A second file, codec_nonfinite_vectors.npz, holds blocks whose groups carry
NaN, +inf, -inf or a range that overflows float32 (hi - lo = inf), next to
finite groups: for K the two nibbles of an int4 byte belong to different
column groups, so torch's packing in float (q[0::2] + 16 q[1::2], then the
uint8 cast) decides whether a NaN quotient zeroes its finite partner.
Run: python tests/golden/make_codec_tie_vectors.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "codec_tie_vectors.npz"
OUT_NONFINITE = Path(__file__).resolve().parent / "codec_nonfinite_vectors.npz"
HEADS, DIM, LAYER = 2, 64, 9


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 values that are exact bf16 -> uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    assert not (u & 0xFFFF).any(), "value not exact in bf16"
    return (u >> 16).astype(np.uint16)


def torch_encode(block: np.ndarray, bits: int, kind: int, layer: int) -> np.ndarray:
    """The op sequence of transport_codec.py:24-36 on one block (b = 1)."""
    src = torch.from_numpy(block.view(np.int16).copy()).view(torch.bfloat16)[None]
    x = src.float()
    b, t, h, d = x.shape
    g = 64
    shape = (b, t // g, g, h, d) if kind == 0 else (b, t, h, d // g, g)
    x = x.reshape(shape)
    axis = 2 if kind == 0 else 4
    low = x.amin(axis, keepdim=True)
    high = x.amax(axis, keepdim=True)
    scale = ((high - low) / ((1 << bits) - 1)).clamp_min(1e-12)
    q = ((x - low) / scale).round().clamp(0, (1 << bits) - 1).reshape(b, -1)
    if bits == 4:
        q = q[:, 0::2] + 16 * q[:, 1::2]
    q = q.to(torch.uint8)
    qb = q.shape[1]
    sb = scale[0].numel() * 4
    width = (qb + 2 * sb + 16 + 15) // 16 * 16
    packet = torch.zeros((b, width), dtype=torch.uint8)
    packet[:, :qb] = q
    packet[:, qb:qb + sb] = scale.contiguous().view(torch.uint8).reshape(b, -1)
    packet[:, qb + sb:qb + 2 * sb] = low.contiguous().view(torch.uint8).reshape(b, -1)
    packet[:, qb + 2 * sb:qb + 2 * sb + 16] = torch.tensor([1, layer, kind, bits], dtype=torch.int32).view(torch.uint8)
    return packet[0].numpy()


def round_bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def tie_group(rng, qmax: int, s: float) -> np.ndarray | None:
    """64 bf16 values: low 0, high qmax*s, the rest at (k + 0.5) * s."""
    hi = np.float32(qmax * s)
    if round_bf16(hi) != hi:
        return None
    ks = rng.integers(0, qmax, 62)
    v = ((ks + 0.5) * s).astype(np.float32)
    ok = round_bf16(v) == v
    v = np.where(ok, v, np.float32(0))
    g = np.concatenate([[np.float32(0), hi], v]).astype(np.float32)
    rng.shuffle(g)
    return g + np.float32(0)  # -0 stays out


def recip_group(rng, qmax: int) -> np.ndarray:
    """64 bf16 values whose low / high set a scale for which many
    (x - low) / scale quotients round to another integer when computed as
    (x - low) * RN(1 / scale)."""
    best, best_hits = None, -1
    for _ in range(400):
        lo = round_bf16(np.float32(rng.normal(0, 1)))
        hi = round_bf16(lo + np.float32(abs(rng.normal(0, 2)) + 0.01))
        s = np.float32(np.float32(hi - lo) / np.float32(qmax))
        if s < np.float32(1e-12):
            continue
        cand = round_bf16(lo + (hi - lo) * rng.random(4000).astype(np.float32))
        cand = cand[(cand >= lo) & (cand <= hi)]
        a = (cand - lo).astype(np.float32)
        exact = np.round(a / s)
        naive = np.round((a * np.float32(np.float32(1) / s)).astype(np.float32))
        hits = cand[exact != naive]
        if hits.size > best_hits:
            best, best_hits = (lo, hi, hits), hits.size
        if best_hits >= 30:
            break
    lo, hi, hits = best
    fill = round_bf16(lo + (hi - lo) * rng.random(62).astype(np.float32))
    vals = np.concatenate([hits[:62], fill[:max(0, 62 - hits.size)]])[:62]
    g = np.concatenate([[lo, hi], vals]).astype(np.float32)
    rng.shuffle(g)
    return g


def make_block(rng, bits: int, kind: int) -> np.ndarray:
    """[128, HEADS, DIM] float32 (bf16-exact), one crafted 64-element group
    per group slot: K groups are (64 tokens, column), V groups (token, head,
    64 dims)."""
    qmax = (1 << bits) - 1
    x = round_bf16(rng.standard_normal((128, HEADS, DIM)).astype(np.float32))
    ngroups = 2 * HEADS * DIM if kind == 0 else 128 * HEADS * (DIM // 64)
    for gi in range(ngroups):
        sel = gi % 8
        if sel in (0, 1, 2, 3):
            s = (1.0, 2.0, 0.5, 0.25)[sel]
            g = tie_group(rng, qmax, s)
            if g is None:
                continue
            if gi % 16 >= 8:
                g = (-g).astype(np.float32)  # mirrored: x - low = (qmax - k - 0.5) * scale, still ties
        elif sel in (4, 5):
            g = recip_group(rng, qmax)
        elif sel == 6:
            g = np.full(64, round_bf16(np.float32(rng.normal())), np.float32)
        else:
            continue  # random N(0,1) group
        if kind == 0:
            tg, col = divmod(gi, HEADS * DIM)
            h, d = divmod(col, DIM)
            x[64 * tg:64 * tg + 64, h, d] = g
        else:
            t, rest = divmod(gi, HEADS * (DIM // 64))
            h, dg = divmod(rest, DIM // 64)
            x[t, h, 64 * dg:64 * dg + 64] = g
    return x


def census(x: np.ndarray, bits: int, kind: int) -> tuple[int, int]:
    """(exact ties, quotients where the reciprocal form rounds differently)."""
    qmax = (1 << bits) - 1
    xf = x.reshape(2, 64, HEADS, DIM) if kind == 0 else x.reshape(128, HEADS, DIM // 64, 64)
    axis = 1 if kind == 0 else 3
    lo = xf.min(axis, keepdims=True)
    hi = xf.max(axis, keepdims=True)
    s = np.maximum(((hi - lo) / np.float32(qmax)).astype(np.float32), np.float32(1e-12))
    a = (xf - lo).astype(np.float32)
    quo = (a / s).astype(np.float32)
    ties = int((quo - np.floor(quo) == 0.5).sum())
    naive = (a * (np.float32(1) / s).astype(np.float32)).astype(np.float32)
    return ties, int((np.round(quo) != np.round(naive)).sum())


def nonfinite_block(rng, kind: int) -> np.ndarray:
    """[128, HEADS, DIM] float32 (bf16-exact) with non-finite groups next to
    finite ones.  K: per (token group, column) patterns cycling over the
    columns, so even and odd columns (the two nibbles of an int4 byte) mix a
    NaN / +inf / -inf / overflowing group with a finite one.  V: every
    fourth (token, head, 64-dim group) gets one such pattern."""
    x = round_bf16(rng.standard_normal((128, HEADS, DIM)).astype(np.float32))
    big = np.float32(3.0e38)  # bf16-exact after rounding; big - (-big) overflows

    def put(g: np.ndarray, pat: int) -> None:
        n = g.size
        i, j = rng.integers(0, n, 2)
        if pat == 0:
            g[i] = np.nan
        elif pat == 1:
            g[i] = np.inf
        elif pat == 2:
            g[i] = -np.inf
        elif pat == 3:
            g[i], g[(i + 1) % n] = np.inf, -np.inf
        elif pat == 4:
            g[i], g[(i + 1) % n] = round_bf16(big), round_bf16(-big)
        elif pat == 5:
            g[i], g[j] = np.inf, np.nan

    if kind == 0:
        for tg in range(2):
            for h in range(HEADS):
                for d in range(DIM):
                    pat = (d + 3 * tg + 5 * h) % 9  # 6..8: finite groups
                    if pat < 6:
                        col = x[64 * tg:64 * tg + 64, h, d].copy()
                        put(col, pat)
                        x[64 * tg:64 * tg + 64, h, d] = col
    else:
        for t in range(128):
            for h in range(HEADS):
                for dg in range(DIM // 64):
                    pat = (t + h + dg) % 8
                    if pat < 6 and t % 4 == 0:
                        seg = x[t, h, 64 * dg:64 * dg + 64].copy()
                        put(seg, pat)
                        x[t, h, 64 * dg:64 * dg + 64] = seg
    return x


def make_nonfinite(rng) -> None:
    blocks, bits_l, kinds, packets = [], [], [], []
    for bits in (8, 4):
        for kind in (0, 1):
            x = nonfinite_block(rng, kind)
            u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
            blk = (u >> 16).astype(np.uint16)  # NaN / inf keep their bf16 patterns
            blocks.append(blk)
            bits_l.append(bits)
            kinds.append(kind)
            packets.append(torch_encode(blk, bits, kind, LAYER))
    np.savez_compressed(OUT_NONFINITE, blocks=np.stack(blocks), bits=np.array(bits_l, np.int32),
                        kinds=np.array(kinds, np.int32), layer=np.int32(LAYER),
                        torch_version=np.array(torch.__version__),
                        **{f"packet_{i}": pk for i, pk in enumerate(packets)})
    print(f"wrote {OUT_NONFINITE}: {len(blocks)} blocks")


def main():
    rng = np.random.default_rng(20261202)
    blocks, bits_l, kinds, packets, ties, recips = [], [], [], [], [], []
    for bits in (8, 4):
        for kind in (0, 1):
            for _ in range(2):
                x = make_block(rng, bits, kind)
                blk = bf16_bits(x)
                blocks.append(blk)
                bits_l.append(bits)
                kinds.append(kind)
                packets.append(torch_encode(blk, bits, kind, LAYER))
                t, r = census(x, bits, kind)
                ties.append(t)
                recips.append(r)
    widths = sorted({p.size for p in packets})
    packed = {f"packets_w{w}": np.stack([p for p in packets if p.size == w]) for w in widths}
    np.savez_compressed(OUT, blocks=np.stack(blocks), bits=np.array(bits_l, np.int32),
                        kinds=np.array(kinds, np.int32), layer=np.int32(LAYER),
                        widths=np.array([p.size for p in packets], np.int64),
                        ties=np.array(ties, np.int64), recip_differs=np.array(recips, np.int64),
                        torch_version=np.array(torch.__version__), **packed)
    print(f"wrote {OUT}: {len(blocks)} blocks, ties {ties}, reciprocal-form differs {recips}")
    make_nonfinite(np.random.default_rng(20261203))


if __name__ == "__main__":
    main()
