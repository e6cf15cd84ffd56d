"""Writes tests/golden/codec_decode_vectors.npz by running the REFERENCE's
decode (secure_infer/kv_offload/optimized_decode.py:5-26, torch-only) on the
CPU of the development container, where the reference's sources are present.

Inputs are packets made by the oracle's restated encoder
(transport_codec.py:22-42 cannot be imported: its module imports vLLM) from
seeded ~N(0,1) bf16 blocks of shape [128, heads, dim=128] for heads 1, 4 and
8 (the configurations' kv-head counts: the parameter layouts K (2, h, d) and
V (128, h, d/64) are only pinned where the head axis is not trivial); for
each (heads, bits, kind) the fixture keeps the packet and decode_into's bf16
output bits.  Keys: heads 1 as block_bf16 / packet_b{bits}_k{kind} /
decoded_b{bits}_k{kind}; heads 4 and 8 (packets and outputs only) with an
h{heads}_ prefix.
The reference file is read from /root/reference (this script only runs where
that tree exists); the fixture is data and travels without it.
Run: python tests/golden/make_codec_vectors.py
"""
import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

REF = Path("/root/reference/secure_infer/kv_offload/optimized_decode.py")
HEADS, DIM = (1, 4, 8), 128


def load_reference_decode():
    spec = importlib.util.spec_from_file_location("ref_optimized_decode", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.decode_into


def main():
    decode_into = load_reference_decode()
    arrays = {}
    for heads in HEADS:
        pre = "" if heads == 1 else f"h{heads}_"
        rng = np.random.default_rng(7 if heads == 1 else 7 + heads)
        x = O.f32_to_bf16(rng.standard_normal((128, heads, DIM), dtype=np.float32))
        if heads == 1:
            arrays["block_bf16"] = x  # the encoder's stability check (heads 1 only)
        for bits in (8, 4):
            for kind in (0, 1):
                pkt = O.codec_encode(x, bits, kind, layer=3)
                qb, sb, width = O.codec_sizes(bits, heads, DIM)
                wire = torch.from_numpy(pkt.copy()).reshape(1, -1)
                dest = torch.zeros((2, 128, heads, DIM), dtype=torch.bfloat16)
                decode_into(wire, dest, torch.tensor([1]), bits, kind, qb, sb)
                out = dest[1].view(torch.int16).numpy().view(np.uint16).copy()
                arrays[f"{pre}packet_b{bits}_k{kind}"] = pkt
                arrays[f"{pre}decoded_b{bits}_k{kind}"] = out
    path = Path(__file__).with_name("codec_decode_vectors.npz")
    np.savez_compressed(path, **arrays)
    print(path, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
