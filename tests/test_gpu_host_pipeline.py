"""GPU tests of the host transfer runtime: host AES-GCM (OpenSSL) + pinned
ring + copy stream feeding the fused reload kernel (secure_infer_h2d_swap,
NativeTransfer), and the D2H batch / group API sealing device blocks that the
host authenticates into its pools (secure_infer_d2h_*, D2HTransfer).

Every comparison is bit-exact against the data that went in, or against the
oracle codec (C restatement) for packets.
"""
import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import oracle as O
from secure_infer_amd import _lib
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEY = bytes(range(0x30, 0x40))
SALT = b"\x11\x22\x33\x44"


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def pools(rng, nblocks, heads, dim):
    """Host K / V pools [nblocks, 128, h, d] of bf16 bit patterns (as int16)."""
    k = torch.from_numpy(np.stack(W.bf16_blocks(rng, nblocks, heads, dim)).view(np.int16))
    v = torch.from_numpy(np.stack(W.bf16_blocks(rng, nblocks, heads, dim)).view(np.int16))
    return k.contiguous(), v.contiguous()


def caches(nslots, heads, dim, fill=0x3C):
    k = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV)
    v = torch.zeros_like(k)
    k.view(torch.uint8).fill_(fill)
    v.view(torch.uint8).fill_(fill)
    return k, v


def test_h2d_pipeline_bf16_layers():
    rng = np.random.default_rng(101)
    heads, dim, ncpu, nslots, nlayers = 4, 128, 12, 24, 6  # more layers than ring slots
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 7, max_record_bytes=shape.record_bytes)
    nt = si.NativeTransfer(sess, shape)
    host_layers, dev_layers, maps = [], [], []
    si.clear_host_ranges()
    try:
        for layer in range(nlayers):
            hk, hv = pools(rng, ncpu, heads, dim)
            si.register_host_range(hk, layer, 0)
            si.register_host_range(hv, layer, 1)
            ck, cv = caches(nslots, heads, dim)
            n = 5 + layer % 3
            cpu_ids = rng.permutation(ncpu)[:n]
            slot_ids = rng.permutation(nslots)[:n]
            mapping = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64))
            nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
            host_layers.append((hk, hv))
            dev_layers.append((ck, cv))
            maps.append((cpu_ids, slot_ids))
        for layer in range(nlayers):
            assert nt.wait_layer(layer) == 0
            (hk, hv), (ck, cv), (cpu_ids, slot_ids) = host_layers[layer], dev_layers[layer], maps[layer]
            kk, vv = host(ck), host(cv)
            for c, sl in zip(cpu_ids, slot_ids):
                assert np.array_equal(kk[sl], hk[c].numpy())
                assert np.array_equal(vv[sl], hv[c].numpy())
            untouched = np.setdiff1d(np.arange(nslots), slot_ids)
            assert (kk[untouched].view(np.uint8) == 0x3C).all()
    finally:
        si.clear_host_ranges()


@pytest.mark.parametrize("bits", [8, 4])
def test_h2d_pipeline_codec(bits):
    rng = np.random.default_rng(111 + bits)
    heads, dim, ncpu, nslots, layer = 4, 128, 6, 10, 3
    shape = si.LayerShape(heads, dim, bits)
    width = shape.record_bytes
    blocks = [W.bf16_blocks(rng, ncpu, heads, dim) for _ in range(2)]
    packets = [np.stack([O.codec_encode(blocks[k][i], bits, k, layer) for i in range(ncpu)])
               for k in range(2)]
    hp = [torch.from_numpy(p).contiguous() for p in packets]  # [ncpu, width] uint8
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=width)
    nt = si.NativeTransfer(sess, shape)
    nt.layer = layer
    ck, cv = caches(nslots, heads, dim)
    cpu_ids = np.array([4, 0, 5, 2])
    slot_ids = np.array([9, 3, 0, 6])
    mapping = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64))
    nt.single_layer_kv_transfer((hp, mapping), (ck, cv))
    assert nt.wait_layer(layer) == 0
    out = [host(ck), host(cv)]
    for k in range(2):
        for c, sl in zip(cpu_ids, slot_ids):
            assert np.array_equal(out[k][sl].view(np.uint16),
                                  O.codec_decode(packets[k][c], heads, dim, bits, k))


@pytest.mark.parametrize("group_blocks", [16, 2])
def test_d2h_store_bf16(group_blocks):
    rng = np.random.default_rng(121 + group_blocks)
    heads, dim, nslots, ncpu, nlayers = 4, 128, 16, 20, 2
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 3, max_record_bytes=shape.record_bytes)
    src, dst, maps = [], [], []
    for _ in range(nlayers):
        k = torch.from_numpy(np.stack(W.bf16_blocks(rng, nslots, heads, dim)).view(np.int16)).to(DEV)
        v = torch.from_numpy(np.stack(W.bf16_blocks(rng, nslots, heads, dim)).view(np.int16)).to(DEV)
        src.append((k, v))
        dst.append((torch.zeros((ncpu, 128, heads, dim), dtype=torch.int16),
                    torch.zeros((ncpu, 128, heads, dim), dtype=torch.int16)))
    n = 7
    slot_ids = rng.permutation(nslots)[:n]
    cpu_ids = rng.permutation(ncpu)[:n]
    mapping = torch.from_numpy(np.stack([slot_ids, cpu_ids], 1).astype(np.int64))
    si.D2HTransfer(sess, shape, group_blocks=group_blocks).store(src, dst, mapping)
    for (k, v), (hk, hv) in zip(src, dst):
        kk, vv = host(k), host(v)
        for sl, c in zip(slot_ids, cpu_ids):
            assert np.array_equal(hk[c].numpy(), kk[sl])
            assert np.array_equal(hv[c].numpy(), vv[sl])
        rest = np.setdiff1d(np.arange(ncpu), cpu_ids)
        assert not hk[rest].numpy().any()


@pytest.mark.parametrize("bits", [4, 8])
def test_d2h_store_codec(bits):
    rng = np.random.default_rng(131 + bits)
    heads, dim, nslots, ncpu, layer = 4, 128, 8, 6, 5
    shape = si.LayerShape(heads, dim, bits)
    width = shape.record_bytes
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=width)
    blocks = [np.stack(W.bf16_blocks(rng, nslots, heads, dim)) for _ in range(2)]
    src = [(torch.from_numpy(blocks[0].view(np.int16)).to(DEV), torch.from_numpy(blocks[1].view(np.int16)).to(DEV))]
    dst = [(torch.zeros((ncpu, width), dtype=torch.uint8), torch.zeros((ncpu, width), dtype=torch.uint8))]
    slot_ids, cpu_ids = np.array([7, 1, 4]), np.array([2, 5, 0])
    mapping = torch.from_numpy(np.stack([slot_ids, cpu_ids], 1).astype(np.int64))
    si.D2HTransfer(sess, shape).store(src, dst, mapping, layers=[layer])
    for k in range(2):
        for sl, c in zip(slot_ids, cpu_ids):
            assert np.array_equal(dst[0][k][c].numpy(), O.codec_encode(blocks[k][sl], bits, k, layer))


def test_d2h_api_semantics():
    L = _lib.load()
    assert L.secure_infer_d2h_batch_end() == 0            # no batch: nothing to do
    assert L.secure_infer_d2h_group_begin(1) == -1        # no batch open
    assert L.secure_infer_d2h_group_end() == 0            # no group open
    assert L.secure_infer_d2h_batch_begin(4) == 1
    assert L.secure_infer_d2h_batch_begin(4) == -1        # nested
    assert L.secure_infer_d2h_group_begin(2) == 1
    assert L.secure_infer_d2h_group_begin(2) == -1        # nested group
    assert L.secure_infer_d2h_batch_device_barrier() == -1  # group still open
    assert L.secure_infer_d2h_batch_end() == -1           # group still open
    assert L.secure_infer_d2h_group_end() == 0
    assert L.secure_infer_d2h_batch_device_barrier() == 0
    assert L.secure_infer_d2h_batch_end() == 0
