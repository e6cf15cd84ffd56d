"""One full-size layer of every benchmark workload through the fused kernels,
at its real record count and cache size (the share / pair layouts the 256-CU
launch takes only appear at these sizes), checked record by record:

* bf16 Llama-3-8B reload: 48 blocks -> 96 records of 262,144 B into 512-slot
  caches (8 kv heads x 128);
* int8 Llama-3-8B reload: 64 blocks -> 128 packets of 147,472 B;
* int4 Qwen2.5-7B reload: 64 blocks -> 128 packets of 40,976 B (4 kv heads),
  two seeded records with one seeded ciphertext byte flipped;
* int4 Llama-3-70B writeback: 256 blocks -> 512 packets of 81,936 B (pairs of
  whole records per workgroup);
* one tensor-parallel rank of Llama-3-70B at TP = 8 (1 kv head x 128 per
  rank): 256 blocks -> 512 bf16 records of 32,768 B reloaded, and 512 int4
  packets of 10,256 B written back (small records: several rounds of pairs).

The bf16 and int4 reload layers also run end to end through the host
pipeline (host pools, NativeTransfer with 16-block causal groups, group
prefetch), and the 70B layer through the D2H store into host packet pools.  Reload ciphertext comes from OpenSSL (the reference's host
AES-128-GCM) over the oracle's packets; outputs must equal the input blocks (bf16) or the
oracle decode of the packets, bit for bit, and every record's status must be
1 except the tampered ones (0, slot zeroed on the device).  Writeback
ciphertext and tags must equal OpenSSL's over the oracle's packets.
"""
import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import oracle as O
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEY = bytes.fromhex("000102030405060708090a0b0c0d0e0f")
SALT = bytes.fromhex("5eed5a17")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def statuses(ww: np.ndarray, n: int, nrec: int) -> np.ndarray:
    st, toff = W.stride(n), W.align32(n)
    return ww.reshape(nrec, st)[:, toff + 16:toff + 20].copy().view(np.uint32).ravel()


@pytest.mark.parametrize("bits,heads,nb", [(0, 8, 48), (8, 8, 64), (4, 4, 64), (0, 1, 256)],
                         ids=["bf16_llama3_8b", "int8_llama3_8b", "int4_qwen2_5_7b", "bf16_llama3_70b_tp8_rank"])
def test_full_size_reload_layer(bits, heads, nb):
    rng = np.random.default_rng(1000 + bits)
    dim, nslots, layer, t0 = 128, 512, 17, 123456
    nrec = 2 * nb
    kinds = [0] * nb + [1] * nb
    blocks = W.bf16_blocks(rng, nrec, heads, dim)
    if bits:
        payloads = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(nrec)]
    else:
        payloads = [blocks[r].view(np.uint8).reshape(-1) for r in range(nrec)]
    n = payloads[0].size
    assert n == (128 * heads * dim * 2 if not bits else si.codec_width(bits, heads, dim))
    wire = W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0)
    tampered = []
    if bits == 4:  # 1 % of a layer's records, rounded up: two seeded records
        tampered = sorted(int(r) for r in rng.choice(nrec, 2, replace=False))
        for r in tampered:
            wire[r * W.stride(n) + int(rng.integers(0, n))] ^= 0x5A
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    slots = dev(np.concatenate([slot_ids, slot_ids]))
    ck = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV)
    cv = torch.zeros_like(ck)
    ck.view(torch.uint8).fill_(0x3C)
    cv.view(torch.uint8).fill_(0x3C)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.empty(nrec * W.align32(n), dtype=torch.uint8, device=DEV) if bits else None
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = dev(wire)
    sess.reload_layer(dw, n, nrec, nb, ck, cv, slots, ticket_base=t0, codec_bits=bits, heads=heads,
                      head_dim=dim, layer=layer, staging=staging, fail_count=fail)
    torch.cuda.synchronize()
    st = statuses(dw.cpu().numpy(), n, nrec)
    want_st = np.ones(nrec, np.uint32)
    want_st[tampered] = 0
    assert np.array_equal(st, want_st)
    assert int(fail.item()) == len(tampered)
    if bits:
        want = np.stack([O.codec_decode(payloads[r], heads, dim, bits, kinds[r]) for r in range(nrec)])
    else:
        want = blocks.copy()
    want[tampered] = 0
    want_dev = dev(want.view(np.int16))
    idx = dev(slot_ids)
    assert torch.equal(ck.index_select(0, idx), want_dev[:nb])
    assert torch.equal(cv.index_select(0, idx), want_dev[nb:])
    for r in tampered:  # what attention would read
        c = ck if r < nb else cv
        s = int(slot_ids[r % nb])
        assert torch.equal(c[s], torch.zeros_like(c[s]))
    untouched = torch.ones(nslots, dtype=torch.bool, device=DEV)
    untouched[idx] = False
    for c in (ck, cv):
        assert bool((c[untouched].view(torch.uint8) == 0x3C).all())


@pytest.mark.parametrize("heads", [8, 1], ids=["llama3_70b", "llama3_70b_tp8_rank"])
def test_full_size_writeback_layer_int4_llama3_70b(heads):
    rng = np.random.default_rng(1070 + heads)
    dim, nb, nslots, layer, bits, t0 = 128, 256, 512, 61, 4, 777000
    nrec = 2 * nb
    kinds = [0] * nb + [1] * nb
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    ck = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV)
    cv = torch.zeros_like(ck)
    data = [W.bf16_blocks(rng, nb, heads, dim) for _ in range(2)]
    idx = dev(slot_ids)
    ck[idx] = dev(data[0].view(np.int16))
    cv[idx] = dev(data[1].view(np.int16))
    n = si.codec_width(bits, heads, dim)
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nb)) * 2, t0)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    staging = torch.empty(nrec * W.align32(n), dtype=torch.uint8, device=DEV)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = dev(wire)
    sess.writeback_layer(dw, n, nrec, nb, ck, cv, dev(np.concatenate([slot_ids, slot_ids])), ticket_base=t0,
                         codec_bits=bits, heads=heads, head_dim=dim, layer=layer, staging=staging,
                         fail_count=fail)
    torch.cuda.synchronize()
    assert int(fail.item()) == 0
    ww = dw.cpu().numpy().reshape(nrec, W.stride(n))
    toff = W.align32(n)
    for r in range(nrec):
        pkt = O.codec_encode(data[kinds[r]][r % nb], bits, kinds[r], layer)
        aad = O.build_gcm_aad(2, kinds[r], layer, r % nb, 0, n, t0 + r)
        c, tag = O.ossl_gcm_encrypt(KEY, O.iv12_from_words(W.record_iv(SALT, t0 + r)), aad, pkt)
        assert np.array_equal(ww[r, :n], c), f"record {r} ciphertext"
        assert ww[r, toff:toff + 16].tobytes() == tag, f"record {r} tag"


@pytest.mark.parametrize("merge", [False, True], ids=["per_group", "merged"])
@pytest.mark.parametrize("bits,heads,nb", [(0, 8, 48), (4, 4, 64)], ids=["bf16_llama3_8b", "int4_qwen2_5_7b"])
def test_full_size_layer_through_the_host_pipeline(bits, heads, nb, merge):
    """A full-size layer end to end: host pools -> NativeTransfer with the
    reference's 16-block causal groups (host OpenSSL seals, group prefetch,
    one DMA per group launch; merged: the layer's groups in one launch from
    one layer prefetch, with one V record corrupted once and repaired by the
    strict retry) -> fused reload into a 512-slot cache; every slot equals its
    host block (bf16) or the oracle decode of its packet, and the other slots
    are untouched."""
    rng = np.random.default_rng(2000 + bits)
    dim, nslots, layer = 128, 512, 9
    shape = si.LayerShape(heads, dim, bits)
    sess = si.GcmSession(KEY, SALT, 31, max_record_bytes=shape.record_bytes)
    blocks = [W.bf16_blocks(rng, nb, heads, dim) for _ in range(2)]
    if bits:
        host = [torch.from_numpy(np.stack([O.codec_encode(blocks[k][i], bits, k, layer) for i in range(nb)]))
                for k in range(2)]
    else:
        host = [torch.from_numpy(np.stack(blocks[k]).view(np.int16)).contiguous() for k in range(2)]
    slots = rng.permutation(nslots)[:nb]
    mapping = torch.from_numpy(np.stack([np.arange(nb), slots], 1).astype(np.int64))
    caches = [torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV) for _ in range(2)]
    for c in caches:
        c.view(torch.uint8).fill_(0x3C)
    si.clear_host_ranges()
    try:
        si.register_host_range(host[0], layer, 0)
        si.register_host_range(host[1], layer, 1)
        nt = si.NativeTransfer(sess, shape, causal_group_blocks=16, merge_groups=merge)
        nt.layer = layer
        if merge:
            si.inject_h2d_tamper(layer=layer, kind=1, host_block=nb // 2 + 1, shots=1)
        nt.single_layer_kv_transfer((host, mapping), caches)
        assert nt.wait_layer(layer) == 0
        torch.cuda.synchronize()
        idx = torch.from_numpy(slots.astype(np.int64)).to(DEV)
        for k in range(2):
            got = caches[k].index_select(0, idx).cpu().numpy().view(np.uint16)
            want = np.stack(blocks[k]) if not bits else np.stack(
                [O.codec_decode(host[k][i].numpy(), heads, dim, bits, k) for i in range(nb)])
            assert np.array_equal(got, want)
            rest = torch.from_numpy(np.setdiff1d(np.arange(nslots), slots).astype(np.int64)).to(DEV)
            assert bool((caches[k].index_select(0, rest).view(torch.uint8) == 0x3C).all())
    finally:
        si.inject_h2d_tamper(shots=0)
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


def test_full_size_writeback_through_the_host_pipeline():
    """One 70B int4 layer stored end to end: 256 blocks x K/V gathered from a
    512-slot cache, quantised, sealed on the device, copied down and
    authenticated by OpenSSL into host packet pools (D2HTransfer, 16-block
    groups); every packet equals the oracle's encoding of its block."""
    rng = np.random.default_rng(3004)
    heads, dim, nslots, nb, layer = 8, 128, 512, 256, 61
    shape = si.LayerShape(heads, dim, 4)
    sess = si.GcmSession(KEY, SALT, 32, max_record_bytes=shape.record_bytes)
    blocks = [W.bf16_blocks(rng, nslots, heads, dim) for _ in range(2)]
    src = [tuple(dev(blocks[k].view(np.int16)) for k in range(2))]
    slots = rng.permutation(nslots)[:nb]
    width = shape.record_bytes
    pools = [(torch.zeros((nb, width), dtype=torch.uint8), torch.zeros((nb, width), dtype=torch.uint8))]
    mapping = torch.from_numpy(np.stack([slots, np.arange(nb)], 1).astype(np.int64))
    si.D2HTransfer(sess, shape, group_blocks=16).store(src, pools, mapping, layers=[layer])
    for k in range(2):
        got = pools[0][k].numpy()
        for i in range(nb):
            assert np.array_equal(got[i], O.codec_encode(blocks[k][slots[i]], 4, k, layer)), (k, i)
