"""Verify-before-release reload (SI_RELOAD_VERIFY_BEFORE_RELEASE): the
reference's order of a fused release -- tag computed and compared before any
plaintext is written, then masked output (ghash.aicpu:623-648; direct
verified release, secure_infer.cpp:5522-5538).

* parity: bf16, int8 and int4 layers with records tampered in the
  ciphertext, the tag and the AAD, and one slot id out of range, give
  exactly what the fused default gives (bit-exact slots, statuses, fail
  counts), and match the oracle;
* order: stopped after its first launch (test hook), the verification has
  written every status and the fail count and has not touched the cache at
  all -- not even the slots of records that verify;
* full-size layers (bf16 Llama-3-8B, int4 Qwen2.5-7B) and the
  allocation-free entry point with the flag.
"""
import ctypes as ct

import numpy as np
import pytest
import torch

import secure_infer_amd as si
from oracle import oracle as O
from secure_infer_amd import _lib
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEY = bytes(range(0xA0, 0xB0))
SALT = b"\x21\x43\x65\x87"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def layer_case(rng, bits, heads, dim, nb, layer, t0, tamper_ct=(), tamper_tag=(), tamper_aad=()):
    kinds = [0] * nb + [1] * nb
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    if bits:
        payloads = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
        want = np.stack([O.codec_decode(payloads[r], heads, dim, bits, kinds[r]) for r in range(2 * nb)])
    else:
        payloads = [blocks[r].view(np.uint8).reshape(-1) for r in range(2 * nb)]
        want = blocks.copy()
    n = payloads[0].size
    wire = W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0)
    st, toff = W.stride(n), W.align32(n)
    for r in tamper_ct:
        wire[r * st + int(rng.integers(0, n))] ^= 0x24
    for r in tamper_tag:
        wire[r * st + toff + int(rng.integers(0, 16))] ^= 0x01
    for r in tamper_aad:
        wire[r * st + toff + 32 + int(rng.integers(0, 64))] ^= 0x80
    bad = sorted(set(tamper_ct) | set(tamper_tag) | set(tamper_aad))
    want[bad] = 0
    return wire, n, want, bad


def run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer, flags, phases=0, noalloc=False):
    caches = [torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV) for _ in range(2)]
    for c in caches:
        c.view(torch.uint8).fill_(0x3C)
    dw = dev(wire)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    slots = dev(np.concatenate([slot_ids, slot_ids]))
    staging = None
    if bits and not noalloc:
        staging = torch.zeros(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
    d = _lib.SiReloadDesc(
        wire=dw.data_ptr(), wire_stride=W.stride(n), bytes=n, nrec=2 * nb, n_k=nb, iv_words=None,
        ticket_base=t0, cache_k=caches[0].data_ptr(), cache_v=caches[1].data_ptr(),
        slot_bytes=caches[0][0].numel() * 2, nslots=nslots, slots=slots.data_ptr(), codec_bits=bits,
        heads=heads, head_dim=dim, layer=layer, staging=None if staging is None else staging.data_ptr(),
        fail_count=fail.data_ptr(), flags=flags)
    L = _lib.load()
    if phases:
        assert L.secure_infer_test_strict_phases(phases) == 0
    fn = L.secure_infer_gpu_reload_layer_noalloc if noalloc else L.secure_infer_gpu_reload_layer
    assert fn(ct.c_void_p(torch.cuda.current_stream().cuda_stream), sess._h, ct.byref(d)) == 0
    torch.cuda.synchronize()
    st = dw.cpu().numpy().reshape(2 * nb, W.stride(n))[:, W.align32(n) + 16:W.align32(n) + 20]
    return caches, st.copy().view("<u4").ravel(), int(fail.item())


@pytest.mark.parametrize("bits,heads,dim", [(0, 2, 128), (8, 4, 128), (4, 4, 64)], ids=["bf16", "int8", "int4"])
def test_strict_release_matches_fused_and_oracle(bits, heads, dim):
    rng = np.random.default_rng(9100 + bits)
    nb, nslots, layer, t0 = 9, 32, 4, 41000 + bits
    wire, n, want, bad = layer_case(rng, bits, heads, dim, nb, layer, t0, tamper_ct=(1, 12), tamper_tag=(5,),
                                    tamper_aad=(16,))
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    slot_ids[7] = nslots + 3  # out of range: records 7 and 16 fail, nothing touched
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    fused = run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer, 0)
    strict = run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer,
                 si.gcm.SI_RELOAD_VERIFY_BEFORE_RELEASE)
    failed = sorted(set(bad) | {7, nb + 7})
    want_st = np.ones(2 * nb, np.uint32)
    want_st[failed] = 0
    for name, (caches, st, fail) in (("fused", fused), ("strict", strict)):
        assert np.array_equal(st, want_st), name
        assert fail == len(failed), name
    assert torch.equal(fused[0][0], strict[0][0]) and torch.equal(fused[0][1], strict[0][1])
    caches = strict[0]
    for r in range(2 * nb):
        i = r % nb
        if i == 7:
            continue
        got = caches[r // nb][int(slot_ids[i])].cpu().numpy().view(np.uint16)
        assert np.array_equal(got, want[r]), r
    used = [int(x) for x in slot_ids if x < nslots]
    untouched = torch.ones(nslots, dtype=torch.bool, device=DEV)
    untouched[used] = False
    for c in caches:
        assert bool((c[untouched].view(torch.uint8) == 0x3C).all())


@pytest.mark.parametrize("bits", [0, 4], ids=["bf16", "int4"])
def test_verification_writes_nothing_before_release(bits):
    """The first launch alone: statuses and the fail count are final, the
    cache is byte for byte what it was (0x3C), also where records verify."""
    rng = np.random.default_rng(9200 + bits)
    heads, dim, nb, nslots, layer, t0 = 4, 128, 6, 20, 2, 42000 + bits
    wire, n, want, bad = layer_case(rng, bits, heads, dim, nb, layer, t0, tamper_ct=(2,), tamper_tag=(9,))
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    caches, st, fail = run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer,
                           si.gcm.SI_RELOAD_VERIFY_BEFORE_RELEASE, phases=1)
    want_st = np.ones(2 * nb, np.uint32)
    want_st[bad] = 0
    assert np.array_equal(st, want_st) and fail == len(bad)
    for c in caches:
        assert bool((c.view(torch.uint8) == 0x3C).all()), "the verification wrote into the cache"
    # the whole sequence then releases exactly the verified records
    caches, st, fail = run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer,
                           si.gcm.SI_RELOAD_VERIFY_BEFORE_RELEASE)
    assert np.array_equal(st, want_st) and fail == len(bad)
    idx = dev(slot_ids)
    wd = dev(want.view(np.int16))
    assert torch.equal(caches[0].index_select(0, idx), wd[:nb])
    assert torch.equal(caches[1].index_select(0, idx), wd[nb:])


@pytest.mark.parametrize("bits,heads,nb", [(0, 8, 48), (4, 4, 64)], ids=["bf16_llama3_8b", "int4_qwen2_5_7b"])
def test_strict_release_full_size_layer(bits, heads, nb):
    rng = np.random.default_rng(9300 + bits)
    dim, nslots, layer, t0 = 128, 512, 11, 43000
    wire, n, want, bad = layer_case(rng, bits, heads, dim, nb, layer, t0, tamper_ct=(3, nb + 40))
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    caches, st, fail = run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer,
                           si.gcm.SI_RELOAD_VERIFY_BEFORE_RELEASE)
    want_st = np.ones(2 * nb, np.uint32)
    want_st[bad] = 0
    assert np.array_equal(st, want_st) and fail == len(bad)
    idx = dev(slot_ids)
    wd = dev(want.view(np.int16))
    assert torch.equal(caches[0].index_select(0, idx), wd[:nb])
    assert torch.equal(caches[1].index_select(0, idx), wd[nb:])


def test_strict_release_through_the_allocation_free_entry():
    rng = np.random.default_rng(9400)
    bits, heads, dim, nb, nslots, layer, t0 = 8, 2, 128, 5, 16, 6, 44000
    wire, n, want, bad = layer_case(rng, bits, heads, dim, nb, layer, t0, tamper_aad=(6,))
    slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    caches, st, fail = run(sess, wire, n, nb, nslots, slot_ids, t0, bits, heads, dim, layer,
                           si.gcm.SI_RELOAD_VERIFY_BEFORE_RELEASE, noalloc=True)
    want_st = np.ones(2 * nb, np.uint32)
    want_st[bad] = 0
    assert np.array_equal(st, want_st) and fail == len(bad)
    idx = dev(slot_ids)
    wd = dev(want.view(np.int16))
    assert torch.equal(caches[0].index_select(0, idx), wd[:nb])
    assert torch.equal(caches[1].index_select(0, idx), wd[nb:])


def test_unknown_reload_flags_are_refused():
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=1024)
    wire = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    cache = torch.zeros((2, 128, 2, 2), dtype=torch.int16, device=DEV)
    slots = torch.zeros(2, dtype=torch.int64, device=DEV)
    d = _lib.SiReloadDesc(wire=wire.data_ptr(), wire_stride=W.stride(1024), bytes=1024, nrec=2, n_k=1,
                          iv_words=None, ticket_base=1, cache_k=cache.data_ptr(), cache_v=cache.data_ptr(),
                          slot_bytes=1024, nslots=2, slots=slots.data_ptr(), codec_bits=0, heads=0, head_dim=0,
                          layer=0, staging=None, fail_count=None, flags=2)
    L = _lib.load()
    assert L.secure_infer_gpu_reload_layer(ct.c_void_p(torch.cuda.current_stream().cuda_stream), sess._h,
                                           ct.byref(d)) == -1
