"""GPU tests of the reference's failure and ordering contract on the host
transfer path:

* strict retry (secure_infer.cpp:7303-7333): a record whose sealed bytes are
  corrupted once is re-sealed from the host copy and the layer authenticates;
  corrupted twice, the layer fails and the record's slot reads as zeros; a
  destroyed session retries nothing and leaves no prefetched records;
* ids outside the host pool or the device cache refuse the swap before any
  work, in both directions, and leave both sides untouched;
* a writeback record over an out-of-range slot carries a tag that cannot
  verify, whether or not the caller passes a fail counter (codec and bf16);
* D2H records corrupted before host authentication are zeroed and fail the
  batch (PIPE_GCM_TAMPER_D2H, :2451-2467);
* work on a side stream is ordered against the caller's stream;
* the mixed codec policy across reload and writeback (transport_codec.py:18-19);
* records sealed at the reference's tickets for (group, kind, block)
  (native_layerwise.py:96-112) authenticate in one fused launch.

Zeroed slots are checked on the device (torch.equal against zeros), the way
attention would read them.
"""
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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def pools(rng, nblocks, heads, dim):
    return [torch.from_numpy(np.ascontiguousarray(W.bf16_blocks(rng, nblocks, heads, dim).view(np.int16)))
            for _ in range(2)]


def caches(nslots, heads, dim, fill=0x3C):
    out = []
    for _ in range(2):
        c = torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV)
        c.view(torch.uint8).fill_(fill)
        out.append(c)
    return out


def zero_on_device(t: torch.Tensor) -> bool:
    return bool(torch.equal(t, torch.zeros_like(t)))


@pytest.fixture
def ranges():
    si.clear_host_ranges()
    yield
    si.clear_host_ranges()
    si.inject_h2d_tamper(shots=0)
    si.inject_d2h_tamper(shots=0)


def reload_with_tamper(shots, streams=None, seed=301):
    rng = np.random.default_rng(seed)
    heads, dim, ncpu, nslots, layer = 4, 128, 10, 24, 5
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 11, max_record_bytes=shape.record_bytes)
    hk, hv = pools(rng, ncpu, heads, dim)
    si.register_host_range(hk, layer, 0)
    si.register_host_range(hv, layer, 1)
    ck, cv = caches(nslots, heads, dim)
    cpu_ids = rng.permutation(ncpu)[:6]
    slot_ids = rng.permutation(nslots)[:6]
    mapping = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64))
    target = int(cpu_ids[2])
    si.inject_h2d_tamper(layer=layer, kind=1, host_block=target, shots=shots)
    nt = si.NativeTransfer(sess, shape, streams=streams)
    nt.layer = layer
    nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
    rc = nt.wait_layer(layer)
    torch.cuda.synchronize()
    return rc, (hk, hv), (ck, cv), cpu_ids, slot_ids, target


def test_strict_retry_recovers_a_one_shot_fault(ranges):
    t_before = si.new_transfer_ticket()
    rc, (hk, hv), (ck, cv), cpu_ids, slot_ids, _ = reload_with_tamper(shots=1)
    assert rc == 0
    for c, s in zip(cpu_ids, slot_ids):
        assert torch.equal(ck[s].cpu(), hk[c]) and torch.equal(cv[s].cpu(), hv[c])
    # 12 records plus one re-seal under a fresh ticket
    assert si.new_transfer_ticket() - t_before == 12 + 1 + 1


def test_strict_retry_fails_a_persistent_fault(ranges):
    rc, (hk, hv), (ck, cv), cpu_ids, slot_ids, target = reload_with_tamper(shots=2)
    assert rc == -1
    for c, s in zip(cpu_ids, slot_ids):
        assert torch.equal(ck[s].cpu(), hk[c])
        if c == target:
            assert zero_on_device(cv[s])
        else:
            assert torch.equal(cv[s].cpu(), hv[c])


def test_destroyed_session_leaves_no_prefetch_and_no_retry(ranges):
    """Destroying a session drops its unconsumed prefetches (a later session,
    possibly at the same address, must not consume records sealed under the
    old key) and leaves its observed swaps without retry: a record that
    failed once then fails its layer's wait."""
    from secure_infer_amd import _lib
    rng = np.random.default_rng(311)
    heads, dim, ncpu, nslots, layer = 4, 128, 10, 24, 5
    shape = si.LayerShape(heads, dim)
    hk, hv = pools(rng, ncpu, heads, dim)
    si.register_host_range(hk, layer, 0)
    si.register_host_range(hv, layer, 1)
    ck, cv = caches(nslots, heads, dim)
    cpu_ids = rng.permutation(ncpu)[:6]
    slot_ids = rng.permutation(nslots)[:6]
    mapping = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64))
    L = _lib.load()
    sess = si.GcmSession(KEY, SALT, 12, max_record_bytes=shape.record_bytes)
    nt = si.NativeTransfer(sess, shape, pipeline_seal=False)
    assert nt.prefetch_kv_transfer(((hk, hv), mapping), layer + 1)
    target = int(cpu_ids[2])
    si.inject_h2d_tamper(layer=layer, kind=1, host_block=target, shots=1)
    nt.layer = layer
    nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
    sess.close()
    assert int(L.secure_infer_count_ready_unconsumed_gcm_tickets()) == 0
    assert nt.wait_layer(layer) == -1
    s = int(slot_ids[2])
    assert zero_on_device(cv[s])
    # A new session serves the same layer normally.
    sess2 = si.GcmSession(KEY, SALT, 13, max_record_bytes=shape.record_bytes)
    nt2 = si.NativeTransfer(sess2, shape)
    nt2.layer = layer
    ck2, cv2 = caches(nslots, heads, dim)
    nt2.single_layer_kv_transfer(((hk, hv), mapping), (ck2, cv2))
    assert nt2.wait_layer(layer) == 0
    for c, sl in zip(cpu_ids, slot_ids):
        assert torch.equal(ck2[sl].cpu(), hk[c]) and torch.equal(cv2[sl].cpu(), hv[c])


def test_side_stream_reload_reports_failure(ranges):
    side = torch.cuda.Stream()
    rc, _, (ck, cv), cpu_ids, slot_ids, target = reload_with_tamper(shots=2, streams=[side], seed=302)
    assert rc == -1
    s = int(slot_ids[list(cpu_ids).index(target)])
    assert zero_on_device(cv[s])


def test_wire_transfer_on_side_stream_orders_its_counter(ranges):
    """Device-resident records on a side stream while the caller's stream is
    busy: the fail counter and slot table are made on the side stream, which
    first waits for the caller's stream, so the tamper count survives."""
    rng = np.random.default_rng(303)
    heads, dim, nb, nslots, layer = 2, 128, 4, 12, 0
    shape = si.LayerShape(heads, dim)
    n = shape.record_bytes
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    wire = W.build_wire(KEY, SALT, [b.view(np.uint8).reshape(-1) for b in blocks], [0] * nb + [1] * nb,
                        layer, list(range(nb)) * 2, 4000)
    wire[(nb + 2) * W.stride(n) + 7] ^= 0x40
    slot_ids = rng.permutation(nslots)[:nb]
    mapping = torch.from_numpy(np.stack([np.arange(nb), slot_ids], 1).astype(np.int64))
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    ck, cv = caches(nslots, heads, dim)
    dw = dev(wire)
    busy = torch.randn((4096, 4096), device=DEV)
    for _ in range(4):
        busy = busy @ busy  # keep the caller's stream occupied
        busy /= busy.norm()
    side = torch.cuda.Stream()
    nt = si.NativeTransfer(sess, shape, stream=side)
    nt.single_layer_wire_transfer((dw, mapping), (ck, cv), ticket_base=4000)
    assert nt.wait_layer(0) == -1
    assert zero_on_device(cv[int(slot_ids[2])])


def test_h2d_refuses_ids_outside_the_pools(ranges):
    rng = np.random.default_rng(304)
    heads, dim, ncpu, nslots = 2, 64, 4, 6
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=shape.record_bytes)
    hk, hv = pools(rng, ncpu, heads, dim)
    ck, cv = caches(nslots, heads, dim)
    nt = si.NativeTransfer(sess, shape)
    t_before = si.new_transfer_ticket()
    for bad in ([[0, 1], [ncpu, 2]], [[0, nslots]], [[-1, 0]], [[1, -2]]):
        with pytest.raises(RuntimeError):
            nt.single_layer_kv_transfer(((hk, hv), torch.tensor(bad, dtype=torch.int64)), (ck, cv))
    torch.cuda.synchronize()
    assert si.new_transfer_ticket() == t_before + 1  # nothing was sealed
    for c in (ck, cv):
        assert bool((c.view(torch.uint8) == 0x3C).all())


def d2h_setup(rng, heads, dim, nslots, ncpu, bits=0):
    shape = si.LayerShape(heads, dim, bits)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=shape.record_bytes)
    data = [W.bf16_blocks(rng, nslots, heads, dim) for _ in range(2)]
    src = [(dev(data[0].view(np.int16)), dev(data[1].view(np.int16)))]
    width = shape.record_bytes
    if bits:
        dst = [tuple(torch.full((ncpu, width), 0x5A, dtype=torch.uint8) for _ in range(2))]
    else:
        dst = [tuple(torch.full((ncpu, 128, heads, dim), 0x5A5A, dtype=torch.int16) for _ in range(2))]
    return shape, sess, data, src, dst


@pytest.mark.parametrize("bad", ["slot_high", "slot_negative", "host_high"])
def test_d2h_refuses_ids_outside_the_pools(ranges, bad):
    rng = np.random.default_rng(305)
    heads, dim, nslots, ncpu = 2, 64, 6, 5
    shape, sess, data, src, dst = d2h_setup(rng, heads, dim, nslots, ncpu)
    m = np.array([[1, 0], [2, 3], [4, 1]], np.int64)
    if bad == "slot_high":
        m[1, 0] = nslots
    elif bad == "slot_negative":
        m[2, 0] = -1
    else:
        m[0, 1] = ncpu
    before = [d.clone() for d in dst[0]]
    with pytest.raises(RuntimeError):
        si.D2HTransfer(sess, shape).store(src, dst, torch.from_numpy(m), layers=[0])
    for d, b in zip(dst[0], before):
        assert torch.equal(d, b)  # no pool byte touched


@pytest.mark.parametrize("bits", [8, 4, 0])
def test_writeback_bad_slot_tag_never_verifies(ranges, bits):
    """fail_count = NULL: the record over an out-of-range slot still cannot be
    authenticated by the host (its tag is the complement of the true one and
    a codec packet encodes zeros, never stale staging bytes)."""
    rng = np.random.default_rng(306 + bits)
    heads, dim, nslots, layer, nb = 8, 128, 8, 3, 3
    shape = si.LayerShape(heads, dim, bits)
    n = shape.record_bytes
    data = [W.bf16_blocks(rng, nslots, heads, dim) for _ in range(2)]
    ck, cv = dev(data[0].view(np.int16)), dev(data[1].view(np.int16))
    slots = np.array([5, nslots + 7, 1, 0, 2, -4], np.int64)  # K record 1 and V record 2 out of range
    kinds = [0] * nb + [1] * nb
    ticket0 = 8100 + bits
    wire = W.wire_aads(KEY, SALT, n, kinds, layer, list(range(nb)) * 2, ticket0)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    stage = torch.full((2 * nb * W.align32(n),), 0xA5, dtype=torch.uint8, device=DEV) if bits else None
    dw = dev(wire)
    sess.writeback_layer(dw, n, 2 * nb, nb, ck, cv, dev(slots), ticket_base=ticket0, codec_bits=bits,
                         heads=heads, head_dim=dim, layer=layer, staging=stage)
    torch.cuda.synchronize()
    ww = dw.cpu().numpy()
    st, toff = W.stride(n), W.align32(n)
    for r in range(2 * nb):
        o = r * st
        iv12 = O.iv12_from_words(W.record_iv(SALT, ticket0 + r))
        aad = ww[o + toff + 32:o + toff + 96].tobytes()
        ok, pt = O.ossl_gcm_decrypt(KEY, iv12, aad, ww[o:o + n], ww[o + toff:o + toff + 16].tobytes())
        if r in (1, 5):
            assert not ok, f"record {r} over a bad slot verified"
            if bits:  # the packet under the poisoned tag encodes zeros, not stale staging bytes
                zero_block = np.zeros((128, heads, dim), np.uint16)
                assert np.array_equal(stage.cpu().numpy()[r * toff:r * toff + n],
                                      O.codec_encode(zero_block, bits, kinds[r], layer))
        else:
            assert ok, f"record {r} failed"
            block = data[kinds[r]][slots[r]]
            want = O.codec_encode(block, bits, kinds[r], layer) if bits else block.view(np.uint8).reshape(-1)
            assert np.array_equal(pt, want)


def test_d2h_tamper_is_rejected_and_zeroed(ranges):
    rng = np.random.default_rng(307)
    heads, dim, nslots, ncpu = 2, 64, 6, 5
    shape, sess, data, src, dst = d2h_setup(rng, heads, dim, nslots, ncpu)
    m = torch.tensor([[1, 0], [2, 3]], dtype=torch.int64)
    si.inject_d2h_tamper(1)
    with pytest.raises(RuntimeError):
        si.D2HTransfer(sess, shape).store(src, dst, m, layers=[0])
    # exactly one of the four records (K/V x 2) was corrupted and zeroed
    zeroed = sum(int(not dst[0][k][c].any()) for k in range(2) for c in (0, 3))
    assert zeroed == 1
    si.inject_d2h_tamper(0)
    si.D2HTransfer(sess, shape).store(src, dst, m, layers=[0])
    for k in range(2):
        for s, c in ((1, 0), (2, 3)):
            assert np.array_equal(dst[0][k][c].numpy().view(np.uint16), data[k][s])


def test_mixed_codec_reload_and_writeback(ranges):
    """Three layers under the mixed policy: int8 on layer 0, int4 on layers
    1-2.  Writeback packets equal the oracle encoder at each layer's bits and
    the reload decodes them bit-exactly into the paged cache."""
    rng = np.random.default_rng(308)
    heads, dim, nslots, ncpu, nlayers = 4, 128, 10, 8, 3
    shape = si.LayerShape(heads, dim, codec="mixed", layers=nlayers)
    assert [shape.bits_for(l) for l in range(nlayers)] == [8, 4, 4]
    sess = si.GcmSession(KEY, SALT, 2, max_record_bytes=shape.record_bytes_for(0))
    data = [[W.bf16_blocks(rng, nslots, heads, dim) for _ in range(2)] for _ in range(nlayers)]
    src = [(dev(d[0].view(np.int16)), dev(d[1].view(np.int16))) for d in data]
    dst = [tuple(torch.zeros((ncpu, shape.record_bytes_for(l)), dtype=torch.uint8) for _ in range(2))
           for l in range(nlayers)]
    for l in range(nlayers):
        for k in range(2):
            si.register_host_range(dst[l][k], l, k)
    slot_ids = np.array([7, 2, 9, 0])
    cpu_ids = np.array([3, 0, 6, 1])
    si.D2HTransfer(sess, shape).store(src, dst, torch.from_numpy(np.stack([slot_ids, cpu_ids], 1)))
    for l in range(nlayers):
        bits = shape.bits_for(l)
        for k in range(2):
            for s, c in zip(slot_ids, cpu_ids):
                assert np.array_equal(dst[l][k][c].numpy(), O.codec_encode(data[l][k][s], bits, k, l))
    nt = si.NativeTransfer(sess, shape)
    back = [caches(nslots, heads, dim) for _ in range(nlayers)]
    new_slots = np.array([1, 8, 4, 5])
    for l in range(nlayers):
        nt.single_layer_kv_transfer((dst[l], torch.from_numpy(np.stack([cpu_ids, new_slots], 1))), back[l])
    for l in range(nlayers):
        assert nt.wait_layer(l) == 0
        bits = shape.bits_for(l)
        for k in range(2):
            out = back[l][k].cpu().numpy().view(np.uint16)
            for c, s in zip(cpu_ids, new_slots):
                assert np.array_equal(out[s], O.codec_decode(dst[l][k][c].numpy(), heads, dim, bits, k))


def test_reference_ticket_order_layer_authenticates(ranges):
    """A 48-block layer (LOAD_CHUNK 2048 -> groups of 16) whose records were
    sealed by OpenSSL at the reference's tickets for (group from the tail,
    kind, block), reloaded in one fused launch with per-record IV words."""
    rng = np.random.default_rng(309)
    heads, dim, nb, nslots, layer, t0 = 8, 128, 48, 512, 6, 70000
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    order = si.reference_ticket_order(nb, 16)
    ticket = {kb: t0 + i for i, kb in enumerate(order)}
    n = 128 * heads * dim * 2
    st, toff = W.stride(n), W.align32(n)
    wire = np.zeros(2 * nb * st, np.uint8)
    ivw = np.zeros((2 * nb, 4), np.uint32)
    for r in range(2 * nb):
        kind, b = divmod(r, nb)
        t = ticket[(kind, b)]
        ivw[r] = W.record_iv(SALT, t)
        aad = O.build_gcm_aad(1, kind, layer, b, 0, n, t)
        c, tag = O.ossl_gcm_encrypt(KEY, O.iv12_from_words(ivw[r]), aad, blocks[r].view(np.uint8).reshape(-1))
        wire[r * st:r * st + n] = c
        wire[r * st + toff:r * st + toff + 16] = np.frombuffer(tag, np.uint8)
        wire[r * st + toff + 32:r * st + toff + 96] = np.frombuffer(aad, np.uint8)
    slot_ids = rng.permutation(nslots)[:nb]
    mapping = torch.from_numpy(np.stack([np.arange(nb), slot_ids], 1).astype(np.int64))
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    ck, cv = caches(nslots, heads, dim)
    nt = si.NativeTransfer(sess, si.LayerShape(heads, dim))
    nt.layer = layer
    nt.single_layer_wire_transfer((dev(wire), mapping), (ck, cv), iv_words_dev=dev(ivw))
    assert nt.wait_layer(layer) == 0
    want = dev(blocks.view(np.int16))
    idx = dev(slot_ids.astype(np.int64))
    assert torch.equal(ck.index_select(0, idx), want[:nb])
    assert torch.equal(cv.index_select(0, idx), want[nb:])


@pytest.mark.parametrize("slices,stripe", [(1, False), (2, True), (2, False)])
def test_causal_groups_through_the_host_pipeline(ranges, slices, stripe):
    """NativeTransfer with 16-block causal groups over 41 host blocks, on one
    stream, striped over two slice streams (native_layerwise.py:113-129) or
    given two slice streams without striping:
    every block lands bit-exactly and tickets advance by one per record, plus
    one for a V record sealed with a one-shot fault and sealed again by the
    strict retry."""
    rng = np.random.default_rng(310 + slices)
    heads, dim, ncpu, nslots, layer = 2, 128, 41, 64, 1
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 5, max_record_bytes=shape.record_bytes)
    hk, hv = pools(rng, ncpu, heads, dim)
    si.register_host_range(hk, layer, 0)
    si.register_host_range(hv, layer, 1)
    ck, cv = caches(nslots, heads, dim)
    slot_ids = rng.permutation(nslots)[:ncpu]
    mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
    streams = None if slices == 1 else [torch.cuda.current_stream(), torch.cuda.Stream()]
    nt = si.NativeTransfer(sess, shape, streams=streams, causal_group_blocks=16, stripe=stripe)
    nt.layer = layer
    si.inject_h2d_tamper(layer=layer, kind=1, host_block=30, shots=1)
    t_before = si.new_transfer_ticket()
    nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
    assert nt.layer == layer + 1
    assert nt.wait_layer(layer) == 0
    assert si.new_transfer_ticket() - t_before == 2 * ncpu + 1 + 1
    idx = dev(slot_ids.astype(np.int64))
    assert torch.equal(ck.index_select(0, idx).cpu(), hk) and torch.equal(cv.index_select(0, idx).cpu(), hv)


@pytest.mark.parametrize("shots,rc_want", [(1, 0), (2, -1)], ids=["one_shot", "persistent"])
def test_ungrouped_swaps_are_observed(ranges, shots, rc_want):
    """Swaps issued outside a layer group, with no fail counter, are observed
    like grouped ones (the reference observes its unbatched copies too,
    secure_infer.cpp:7036-7052): a record corrupted once is re-sealed and the
    layer authenticates; corrupted on the retry too, the layer's wait returns
    -1 and the slot reads as zeros."""
    import ctypes as ct

    from secure_infer_amd import _lib
    rng = np.random.default_rng(331 + shots)
    heads, dim, ncpu, nslots, layer = 2, 128, 8, 16, 7
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 21, max_record_bytes=shape.record_bytes)
    hk, hv = pools(rng, ncpu, heads, dim)
    si.register_host_range(hk, layer, 0)
    si.register_host_range(hv, layer, 1)
    ck, cv = caches(nslots, heads, dim)
    cpu_ids = rng.permutation(ncpu)[:5]
    slot_ids = rng.permutation(nslots)[:5]
    mapping = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64))
    target = int(cpu_ids[3])
    si.inject_h2d_tamper(layer=layer, kind=0, host_block=target, shots=shots)
    L = _lib.load()
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    bb = hk[0].numel() * 2
    for pool, cache, kind in ((hk, ck, 0), (hv, cv, 1)):
        assert L.secure_infer_h2d_swap(stream, sess._h, ct.c_void_p(pool.data_ptr()), bb, ncpu,
                                       ct.c_void_p(cache.data_ptr()), bb, nslots,
                                       ct.c_void_p(mapping.data_ptr()), 5, kind, layer, 0, heads, dim, None) == 0
    assert si.NativeTransfer(sess, shape).wait_layer(layer) == rc_want
    torch.cuda.synchronize()
    for c, s in zip(cpu_ids, slot_ids):
        assert torch.equal(cv[s].cpu(), hv[c])
        if c == target and rc_want == -1:
            assert zero_on_device(ck[s])
        else:
            assert torch.equal(ck[s].cpu(), hk[c])


def test_session_destroy_refuses_while_another_thread_holds_it(ranges):
    """A thread's layer group (an H2D launch not yet issued) or D2H batch (a
    job not yet issued) names its session: destroying the session from
    another thread returns -1 and leaves it usable; once the work is issued,
    destroy succeeds."""
    import ctypes as ct
    import threading

    from secure_infer_amd import _lib
    rng = np.random.default_rng(341)
    heads, dim, ncpu, nslots, layer = 2, 128, 6, 12, 3
    shape = si.LayerShape(heads, dim)
    L = _lib.load()
    bb = 128 * heads * dim * 2
    hk, hv = pools(rng, ncpu, heads, dim)
    si.register_host_range(hk, layer, 0)
    si.register_host_range(hv, layer, 1)
    ck, cv = caches(nslots, heads, dim)
    mapping = torch.from_numpy(np.stack([np.arange(4), rng.permutation(nslots)[:4]], 1).astype(np.int64))
    back = torch.stack([mapping[:, 1], mapping[:, 0]], 1).contiguous()
    for direction in ("h2d", "d2h"):
        sess = si.GcmSession(KEY, SALT, 40, max_record_bytes=shape.record_bytes)
        opened, release, closed = threading.Event(), threading.Event(), threading.Event()
        rcs = []

        def holder():
            stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
            if direction == "h2d":
                rcs.append(L.secure_infer_h2d_layer_group_begin(8))
                rcs.append(L.secure_infer_h2d_swap(stream, sess._h, ct.c_void_p(hk.data_ptr()), bb, ncpu,
                                                   ct.c_void_p(ck.data_ptr()), bb, nslots,
                                                   ct.c_void_p(mapping.data_ptr()), 4, 0, layer, 0, heads, dim,
                                                   None))
                opened.set()
                release.wait(60)
                rcs.append(L.secure_infer_h2d_layer_group_end())
                rcs.append(L.secure_infer_recovery_wait_layer_authentication(layer))
            else:
                rcs.append(L.secure_infer_d2h_batch_begin(4) - 1)
                rcs.append(L.secure_infer_d2h_group_begin(4) - 1)
                rcs.append(L.secure_infer_d2h_swap(stream, sess._h, ct.c_void_p(ck.data_ptr()), bb, nslots,
                                                   ct.c_void_p(hv.data_ptr()), bb, ncpu,
                                                   ct.c_void_p(back.data_ptr()), 4, 0, layer, 0, heads, dim))
                rcs.append(L.secure_infer_d2h_group_end())
                opened.set()
                release.wait(60)
                rcs.append(L.secure_infer_d2h_batch_device_barrier())
                rcs.append(L.secure_infer_d2h_batch_end())
            torch.cuda.synchronize()
            closed.set()

        t = threading.Thread(target=holder)
        t.start()
        assert opened.wait(60)
        assert L.secure_infer_gpu_session_destroy(sess._h) == -1, direction  # still held
        release.set()
        assert closed.wait(60)
        t.join(60)
        assert rcs == [0] * len(rcs), (direction, rcs)
        assert L.secure_infer_gpu_session_destroy(sess._h) == 0, direction
        sess._h = ct.c_void_p()  # destroyed here, not by the wrapper
