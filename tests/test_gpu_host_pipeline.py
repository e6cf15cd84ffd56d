"""GPU tests of the host transfer runtime: host AES-GCM (OpenSSL) + pinned
ring + copy stream feeding the fused reload kernel (secure_infer_h2d_swap,
NativeTransfer), and the D2H batch / group API sealing device blocks that the
host authenticates into its pools (secure_infer_d2h_*, D2HTransfer).

Every comparison is bit-exact against the data that went in, or against the
oracle codec (C restatement) for packets.
"""
import ctypes as ct
import os
import time

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


def test_d2h_launch_with_a_ticket_gap():
    """A batch's D2H swaps of one layer share a launch; a ticket reserved by
    someone else between them (here: new_transfer_ticket) makes the launch
    carry explicit per-record IV words.  Host authentication must still pass
    and the pools end bit-exact."""
    rng = np.random.default_rng(151)
    heads, dim, nslots, ncpu = 2, 128, 12, 10
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 6, max_record_bytes=shape.record_bytes)
    k = torch.from_numpy(np.stack(W.bf16_blocks(rng, nslots, heads, dim)).view(np.int16)).to(DEV)
    v = torch.from_numpy(np.stack(W.bf16_blocks(rng, nslots, heads, dim)).view(np.int16)).to(DEV)
    hk = torch.zeros((ncpu, 128, heads, dim), dtype=torch.int16)
    hv = torch.zeros_like(hk)
    m = torch.tensor([[3, 0], [11, 9], [5, 4]], dtype=torch.int64)
    L = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    bb = hk[0].numel() * 2

    def swap(cache, pool, kind):
        return L.secure_infer_d2h_swap(ct.c_void_p(stream), sess._h, ct.c_void_p(cache.data_ptr()), bb, nslots,
                                       ct.c_void_p(pool.data_ptr()), bb, ncpu, ct.c_void_p(m.data_ptr()), 3, kind,
                                       0, 0, heads, dim)

    assert L.secure_infer_d2h_batch_begin(6) > 0
    for cache, pool, kind in ((k, hk, 0), (v, hv, 1)):
        assert L.secure_infer_d2h_group_begin(3) > 0
        assert swap(cache, pool, kind) == 0
        assert L.secure_infer_d2h_group_end() == 0
        si.new_transfer_ticket()  # a gap between the K and the V tickets
    assert L.secure_infer_d2h_batch_device_barrier() == 0
    assert L.secure_infer_d2h_batch_end() == 0
    kk, vv = host(k), host(v)
    for sl, c in m.tolist():
        assert np.array_equal(hk[c].numpy(), kk[sl]) and np.array_equal(hv[c].numpy(), vv[sl])


def test_concurrent_threads_and_streams():
    """Two threads reload different layers through their own streams (own
    rings, workspaces and pending launches) while a third stores a batch
    through the D2H path, all on one session and one worker pool; every
    layer authenticates and every byte lands."""
    import threading
    rng = np.random.default_rng(161)
    heads, dim, ncpu, nslots = 2, 128, 40, 64
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 12, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        layers = _layers(rng, 8, ncpu, heads, dim)
        slot_ids = rng.permutation(nslots)[:ncpu]
        mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
        dst = [caches(nslots, heads, dim) for _ in range(8)]
        src = [tuple(torch.from_numpy(np.stack(W.bf16_blocks(rng, nslots, heads, dim)).view(np.int16)).to(DEV)
                     for _ in range(2)) for _ in range(3)]
        pools_out = [tuple(torch.zeros((ncpu, 128, heads, dim), dtype=torch.int16) for _ in range(2))
                     for _ in range(3)]
        back = torch.stack([mapping[:, 1], mapping[:, 0]], 1).contiguous()
        errors = []

        def reload(first):
            try:
                st = torch.cuda.Stream()
                with torch.cuda.stream(st):
                    nt = si.NativeTransfer(sess, shape, causal_group_blocks=16)
                    nt.layer = first
                    for layer in range(first, first + 4):
                        nt.single_layer_kv_transfer((layers[layer], mapping), dst[layer])
                st.synchronize()
            except Exception as e:  # reported by the main thread
                errors.append(e)

        def store():
            try:
                st = torch.cuda.Stream()
                with torch.cuda.stream(st):
                    si.D2HTransfer(sess, shape, stream=st).store(src, pools_out, back, layers=[20, 21, 22])
                st.synchronize()
            except Exception as e:
                errors.append(e)

        torch.cuda.synchronize()
        threads = [threading.Thread(target=reload, args=(0,)), threading.Thread(target=reload, args=(4,)),
                   threading.Thread(target=store)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
        nt = si.NativeTransfer(sess, shape)
        assert all(nt.wait_layer(layer) == 0 for layer in range(8))
        torch.cuda.synchronize()
        idx = torch.from_numpy(slot_ids.astype(np.int64)).to(DEV)
        for layer in range(8):
            (hk, hv), (ck, cv) = layers[layer], dst[layer]
            assert torch.equal(ck.index_select(0, idx).cpu(), hk) and torch.equal(cv.index_select(0, idx).cpu(), hv)
        for (k, v), (pk, pv) in zip(src, pools_out):
            assert torch.equal(pk, k.index_select(0, idx).cpu()) and torch.equal(pv, v.index_select(0, idx).cpu())
    finally:
        si.clear_host_ranges()


def run_thread_to_exit(fn):
    """Runs fn on a new thread and waits for the OS thread to end: join
    returns once the Python function has returned, and the library's
    thread-local state is destroyed later, at the thread's exit."""
    import threading
    t = threading.Thread(target=fn)
    t.start()
    t.join()
    deadline = time.monotonic() + 60
    while os.path.exists(f"/proc/self/task/{t.native_id}") and time.monotonic() < deadline:
        time.sleep(0.005)


def test_thread_ending_inside_a_group_returns_its_ring_slot():
    """A thread that ends inside a layer group leaves a launch that was never
    issued; its ring slot goes back to the stream's ring (16 slots), so more
    such threads than slots do not starve later swaps on that stream."""
    rng = np.random.default_rng(171)
    heads, dim, ncpu, nslots = 2, 128, 6, 8
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 13, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        hk, hv = pools(rng, ncpu, heads, dim)
        si.register_host_range(hk, 0, 0)
        si.register_host_range(hv, 0, 1)
        ck, cv = caches(nslots, heads, dim)
        st = torch.cuda.Stream()
        L = _lib.load()
        one = torch.tensor([[0, 1]], dtype=torch.int64)
        rcs = []

        def abandon():
            rcs.append(L.secure_infer_h2d_layer_group_begin(2))
            rcs.append(L.secure_infer_h2d_swap(
                ct.c_void_p(st.cuda_stream), sess._h, ct.c_void_p(hk.data_ptr()), hk.stride(0) * 2, ncpu,
                ct.c_void_p(ck.data_ptr()), ck.stride(0) * 2, nslots, ct.c_void_p(one.data_ptr()), 1, 0, 0, 0,
                heads, dim, None))

        for _ in range(20):
            run_thread_to_exit(abandon)
        assert rcs == [0] * 40
        cpu_ids, slot_ids = np.array([5, 0, 3, 2]), np.array([7, 1, 4, 0])
        mapping = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64))
        with torch.cuda.stream(st):
            nt = si.NativeTransfer(sess, shape)
            nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
            assert nt.wait_layer(0) == 0
        kk, vv = host(ck), host(cv)
        for c, sl in zip(cpu_ids, slot_ids):
            assert np.array_equal(kk[sl], hk[c].numpy()) and np.array_equal(vv[sl], hv[c].numpy())
    finally:
        si.clear_host_ranges()


def test_thread_ending_inside_a_d2h_batch():
    """A thread that ends between batch begin and batch end: the launch it
    issued (device barrier) is still verified into the host pool before its
    batch goes, the records never issued are dropped, and later batches run."""
    rng = np.random.default_rng(181)
    heads, dim, nslots, ncpu = 2, 128, 8, 6
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 14, max_record_bytes=shape.record_bytes)
    k = torch.from_numpy(np.stack(W.bf16_blocks(rng, nslots, heads, dim)).view(np.int16)).to(DEV)
    pool = torch.zeros((ncpu, 128, heads, dim), dtype=torch.int16)
    issued = torch.tensor([[3, 1], [6, 4]], dtype=torch.int64)
    dropped = torch.tensor([[0, 0]], dtype=torch.int64)
    L = _lib.load()
    rcs = []

    def swap(mapping, layer):
        rcs.append(L.secure_infer_d2h_group_begin(mapping.shape[0]))
        rcs.append(L.secure_infer_d2h_swap(
            ct.c_void_p(torch.cuda.current_stream().cuda_stream), sess._h, ct.c_void_p(k.data_ptr()),
            k[0].numel() * 2, nslots, ct.c_void_p(pool.data_ptr()), pool[0].numel() * 2, ncpu,
            ct.c_void_p(mapping.data_ptr()), mapping.shape[0], 0, layer, 0, heads, dim))
        rcs.append(L.secure_infer_d2h_group_end())

    def abandon():
        rcs.append(L.secure_infer_d2h_batch_begin(3))
        swap(issued, 0)
        rcs.append(L.secure_infer_d2h_batch_device_barrier())
        swap(dropped, 1)  # pending when the thread ends

    run_thread_to_exit(abandon)
    assert rcs == [1, 1, 0, 0, 0, 1, 0, 0]
    kk = host(k)
    assert np.array_equal(pool[1].numpy(), kk[3]) and np.array_equal(pool[4].numpy(), kk[6])
    assert not pool[0].numpy().any()
    # The runtime still serves a whole batch afterwards.
    dst = [(torch.zeros_like(pool), torch.zeros_like(pool))]
    si.D2HTransfer(sess, shape).store([(k, k)], dst, issued)
    assert np.array_equal(dst[0][1][4].numpy(), kk[6])


D2H_INFLIGHT_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import secure_infer_amd as si
heads, dim, nlayers = 2, 128, 12
shape = si.LayerShape(heads, dim, 4)
sess = si.GcmSession(bytes(16), b"abcd", 0, max_record_bytes=shape.record_bytes)
g = torch.Generator(device="cuda").manual_seed(5)
src = [tuple(torch.randn((16, 128, heads, dim), generator=g, device="cuda").to(torch.bfloat16) for _ in range(2))
       for _ in range(nlayers)]
dst = [tuple(torch.zeros((16, shape.record_bytes), dtype=torch.uint8) for _ in range(2)) for _ in range(nlayers)]
m = torch.stack([torch.arange(16).flip(0), torch.arange(16)], 1).contiguous()
si.D2HTransfer(sess, shape).store(src, dst, m, layers=list(range(nlayers)))
ref = [tuple(torch.zeros_like(t) for t in d) for d in dst]
for layer in range(nlayers):
    si.D2HTransfer(sess, shape).store([src[layer]], [ref[layer]], m, layers=[layer])
assert all(torch.equal(a, b) for d, r in zip(dst, ref) for a, b in zip(d, r))
assert all(bool(t.any()) for d in dst for t in d)
print("done")
"""


def test_d2h_batch_beyond_the_inflight_bound():
    """SECURE_INFER_D2H_INFLIGHT_MB=1: every launch of a 12-layer int4 store
    waits for the previous one's host authentication; the pools equal those
    of one batch per layer."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    env = dict(os.environ, SECURE_INFER_D2H_INFLIGHT_MB="1")
    out = subprocess.run([sys.executable, "-c", D2H_INFLIGHT_SCRIPT, str(Path(__file__).resolve().parent.parent)],
                         env=env, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0 and "done" in out.stdout, out.stderr[-2000:]


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


def _layers(rng, nlayers, ncpu, heads, dim):
    out = []
    for layer in range(nlayers):
        hk, hv = pools(rng, ncpu, heads, dim)
        si.register_host_range(hk, layer, 0)
        si.register_host_range(hv, layer, 1)
        out.append((hk, hv))
    return out


def test_prefetched_records_serve_the_swaps():
    """Ahead-of-demand sealing (secure_infer.cpp:3264-3710): every swap of a
    3-layer reload with 16-block causal groups finds its records sealed, the
    caches end bit-exact, and nothing is left unconsumed."""
    rng = np.random.default_rng(141)
    heads, dim, ncpu, nslots, nlayers = 2, 128, 41, 64, 3
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 9, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        host_layers = _layers(rng, nlayers, ncpu, heads, dim)
        nt = si.NativeTransfer(sess, shape, causal_group_blocks=16)
        slot_ids = rng.permutation(nslots)[:ncpu]
        mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
        before = si.transfer_prefetch_stats()
        for layer in range(nlayers):
            assert nt.prefetch_kv_transfer((host_layers[layer], mapping), layer)
        caches_l = [caches(nslots, heads, dim) for _ in range(nlayers)]
        for layer in range(nlayers):
            nt.single_layer_kv_transfer((host_layers[layer], mapping), caches_l[layer])
        after = si.transfer_prefetch_stats()
        swaps = nlayers * 3 * 2  # groups of 16, 16, 9 blocks, K and V
        served = (after["ready"] - before["ready"]) + (after["busy_fallback"] - before["busy_fallback"])
        assert served == swaps and after["missing_fallback"] == before["missing_fallback"]
        assert int(_lib.load().secure_infer_count_ready_unconsumed_gcm_tickets()) == 0
        idx = torch.from_numpy(slot_ids.astype(np.int64)).to(DEV)
        for layer in range(nlayers):
            assert nt.wait_layer(layer) == 0
            (hk, hv), (ck, cv) = host_layers[layer], caches_l[layer]
            assert torch.equal(ck.index_select(0, idx).cpu(), hk) and torch.equal(cv.index_select(0, idx).cpu(), hv)
    finally:
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


@pytest.mark.parametrize("merge", [False, True], ids=["per_group", "merged"])
def test_reload_layers_one_layer_ahead(merge):
    """reload_layers with lookahead 1 (layer l + 1 sealing while layer l
    copies): 4 layers of 41 blocks in 16-block causal groups, every swap
    served by a prefetch, nothing left unconsumed, exactly 2 x 41 tickets per
    layer, every layer authenticated and bit-exact."""
    rng = np.random.default_rng(147 + int(merge))
    heads, dim, ncpu, nslots, nlayers = 2, 128, 41, 64, 4
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 12, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        host_layers = _layers(rng, nlayers, ncpu, heads, dim)
        nt = si.NativeTransfer(sess, shape, causal_group_blocks=16, merge_groups=merge)
        slot_ids = rng.permutation(nslots)[:ncpu]
        mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
        caches_l = [caches(nslots, heads, dim) for _ in range(nlayers)]
        before = si.transfer_prefetch_stats()
        t0 = si.new_transfer_ticket()
        nt.reload_layers([(host_layers[l], mapping) for l in range(nlayers)], caches_l, lookahead=1)
        assert si.new_transfer_ticket() == t0 + nlayers * 2 * ncpu + 1
        after = si.transfer_prefetch_stats()
        served = (after["ready"] - before["ready"]) + (after["busy_fallback"] - before["busy_fallback"])
        assert served == nlayers * 6 and after["missing_fallback"] == before["missing_fallback"]
        idx = torch.from_numpy(slot_ids.astype(np.int64)).to(DEV)
        for layer in range(nlayers):
            assert nt.wait_layer(layer) == 0
            (hk, hv), (ck, cv) = host_layers[layer], caches_l[layer]
            assert torch.equal(ck.index_select(0, idx).cpu(), hk) and torch.equal(cv.index_select(0, idx).cpu(), hv)
        assert int(_lib.load().secure_infer_count_ready_unconsumed_gcm_tickets()) == 0
    finally:
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


def test_retired_prefetch_falls_back_to_sealing_on_demand():
    rng = np.random.default_rng(142)
    heads, dim, ncpu, nslots = 2, 128, 4, 8
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 1, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        (hk, hv), = _layers(rng, 1, ncpu, heads, dim)
        mapping = torch.tensor([[0, 5], [3, 1]], dtype=torch.int64)
        nt = si.NativeTransfer(sess, shape)
        assert nt.prefetch_kv_transfer(((hk, hv), mapping), 0)
        hk[3].fill_(0x1234)  # host block changed after the prefetch
        si.retire_transfer_prefetches()
        before = si.transfer_prefetch_stats()
        ck, cv = caches(nslots, heads, dim)
        nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
        assert nt.wait_layer(0) == 0
        after = si.transfer_prefetch_stats()
        assert after["missing_fallback"] - before["missing_fallback"] == 2
        assert torch.equal(ck[1].cpu(), hk[3]) and torch.equal(cv[5].cpu(), hv[0])
    finally:
        si.clear_host_ranges()


def test_group_launch_mixes_sources_and_ticket_runs():
    """A layer group's K and V swaps go out as one launch even when the K
    records come from a prefetch buffer and the V records are sealed on
    demand under tickets that do not follow the K tickets (another prefetch
    reserved tickets in between): the launch then carries explicit per-record
    IV words.  A one-shot tamper of a V record is retried from its own
    status word; the caches end bit-exact."""
    rng = np.random.default_rng(144)
    heads, dim, ncpu, nslots, layer = 2, 128, 9, 16, 2
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 5, max_record_bytes=shape.record_bytes)
    L = _lib.load()
    si.clear_host_ranges()
    try:
        hk, hv = pools(rng, ncpu, heads, dim)
        other, _ = pools(rng, ncpu, heads, dim)
        si.register_host_range(hk, layer, 0)
        si.register_host_range(hv, layer, 1)
        si.register_host_range(other, layer + 1, 0)
        ck, cv = caches(nslots, heads, dim)
        cpu_ids = np.array([8, 1, 4, 0, 6])
        slot_ids = np.array([3, 15, 0, 9, 7])
        m = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64)).contiguous()
        stream = torch.cuda.current_stream().cuda_stream
        bb = hk[0].numel() * 2

        def prefetch(pool, kind, lay):
            assert L.secure_infer_h2d_prefetch(sess._h, ct.c_void_p(pool.data_ptr()), bb, ncpu,
                                               ct.c_void_p(m.data_ptr()), len(cpu_ids), kind, lay, 0, heads, dim) == 0

        def swap(pool, cache, kind):
            return L.secure_infer_h2d_swap(ct.c_void_p(stream), sess._h, ct.c_void_p(pool.data_ptr()), bb, ncpu,
                                           ct.c_void_p(cache.data_ptr()), bb, nslots, ct.c_void_p(m.data_ptr()),
                                           len(cpu_ids), kind, layer, 0, heads, dim, None)

        prefetch(hk, 0, layer)
        before = si.transfer_prefetch_stats()
        si.inject_h2d_tamper(layer=layer, kind=1, host_block=4, shots=1)
        assert L.secure_infer_h2d_layer_group_begin(2 * len(cpu_ids)) == 0
        assert swap(hk, ck, 0) == 0
        prefetch(other, 0, layer + 1)  # tickets between the K and the V records
        assert swap(hv, cv, 1) == 0
        assert L.secure_infer_h2d_layer_group_end() == 0
        assert si.NativeTransfer(sess, shape).wait_layer(layer) == 0
        after = si.transfer_prefetch_stats()
        assert after["ready"] + after["busy_fallback"] - before["ready"] - before["busy_fallback"] == 1
        idx = torch.from_numpy(slot_ids.astype(np.int64)).to(DEV)
        cid = torch.from_numpy(cpu_ids.astype(np.int64))
        assert torch.equal(ck.index_select(0, idx).cpu(), hk.index_select(0, cid))
        assert torch.equal(cv.index_select(0, idx).cpu(), hv.index_select(0, cid))
    finally:
        si.inject_h2d_tamper(shots=0)
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


@pytest.mark.parametrize("same_slots", [True, False], ids=["one_copy", "slots_differ"])
def test_group_prefetch_serves_the_group_launch(same_slots):
    """secure_infer_h2d_prefetch_group seals a group's K and V records (and its
    slot ids) into one buffer under tickets K then V.  The group's launch
    takes them in one copy when its slots are the prefetched ones, and falls
    back to separate record and slot-id copies when they are not; either way
    both swaps are served by the prefetch and the caches end bit-exact."""
    rng = np.random.default_rng(145)
    heads, dim, ncpu, nslots, layer = 2, 128, 9, 16, 4
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 6, max_record_bytes=shape.record_bytes)
    L = _lib.load()
    si.clear_host_ranges()
    try:
        hk, hv = pools(rng, ncpu, heads, dim)
        si.register_host_range(hk, layer, 0)
        si.register_host_range(hv, layer, 1)
        ck, cv = caches(nslots, heads, dim)
        cpu_ids = np.array([8, 1, 4, 0, 6])
        slot_ids = np.array([3, 15, 0, 9, 7])
        pre_slots = slot_ids if same_slots else slot_ids[::-1].copy()
        m = torch.from_numpy(np.stack([cpu_ids, slot_ids], 1).astype(np.int64)).contiguous()
        mp = torch.from_numpy(np.stack([cpu_ids, pre_slots], 1).astype(np.int64)).contiguous()
        stream = torch.cuda.current_stream().cuda_stream
        bb = hk[0].numel() * 2
        t0 = si.new_transfer_ticket()
        assert L.secure_infer_h2d_prefetch_group(sess._h, ct.c_void_p(hk.data_ptr()), ct.c_void_p(hv.data_ptr()),
                                                 bb, ncpu, ct.c_void_p(mp.data_ptr()), len(cpu_ids), layer, 0,
                                                 heads, dim) == 0
        assert si.new_transfer_ticket() == t0 + 2 * len(cpu_ids) + 1  # K then V tickets, one run
        before = si.transfer_prefetch_stats()

        def swap(pool, cache, kind):
            return L.secure_infer_h2d_swap(ct.c_void_p(stream), sess._h, ct.c_void_p(pool.data_ptr()), bb, ncpu,
                                           ct.c_void_p(cache.data_ptr()), bb, nslots, ct.c_void_p(m.data_ptr()),
                                           len(cpu_ids), kind, layer, 0, heads, dim, None)

        assert L.secure_infer_h2d_layer_group_begin(2 * len(cpu_ids)) == 0
        assert swap(hk, ck, 0) == 0 and swap(hv, cv, 1) == 0
        assert L.secure_infer_h2d_layer_group_end() == 0
        assert si.NativeTransfer(sess, shape).wait_layer(layer) == 0
        after = si.transfer_prefetch_stats()
        assert after["ready"] + after["busy_fallback"] - before["ready"] - before["busy_fallback"] == 2
        assert after["missing_fallback"] == before["missing_fallback"]
        idx = torch.from_numpy(slot_ids.astype(np.int64)).to(DEV)
        cid = torch.from_numpy(cpu_ids.astype(np.int64))
        assert torch.equal(ck.index_select(0, idx).cpu(), hk.index_select(0, cid))
        assert torch.equal(cv.index_select(0, idx).cpu(), hv.index_select(0, cid))
        untouched = np.setdiff1d(np.arange(nslots), slot_ids)
        assert (host(ck)[untouched].view(np.uint8) == 0x3C).all()
    finally:
        si.inject_h2d_tamper(shots=0)
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


def test_group_prefetch_tamper_is_retried():
    """A record of a group prefetch corrupted after sealing fails once and is
    re-sealed from its host block; the layer authenticates."""
    rng = np.random.default_rng(146)
    heads, dim, ncpu, nslots, layer = 2, 128, 6, 12, 5
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 7, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        hk, hv = pools(rng, ncpu, heads, dim)
        si.register_host_range(hk, layer, 0)
        si.register_host_range(hv, layer, 1)
        ck, cv = caches(nslots, heads, dim)
        mapping = torch.tensor([[5, 2], [0, 11], [3, 7]], dtype=torch.int64)
        si.inject_h2d_tamper(layer=layer, kind=0, host_block=0, shots=1)
        nt = si.NativeTransfer(sess, shape)  # one stream: group prefetches
        nt.layer = layer
        nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
        assert nt.wait_layer(layer) == 0
        for c, sl in mapping.tolist():
            assert torch.equal(ck[sl].cpu(), hk[c]) and torch.equal(cv[sl].cpu(), hv[c])
    finally:
        si.inject_h2d_tamper(shots=0)
        si.clear_host_ranges()


def _codec_layers(rng, nlayers, ncpu, heads, dim, bits):
    """Per layer, host packet pools [ncpu, width] (uint8) encoded by the
    oracle codec from random bf16 blocks, and those blocks."""
    out = []
    for layer in range(nlayers):
        blocks = [W.bf16_blocks(rng, ncpu, heads, dim) for _ in range(2)]
        packets = [torch.from_numpy(np.stack([O.codec_encode(blocks[k][i], bits, k, layer)
                                              for i in range(ncpu)])).contiguous() for k in range(2)]
        si.register_host_range(packets[0], layer, 0)
        si.register_host_range(packets[1], layer, 1)
        out.append((packets, blocks))
    return out


@pytest.mark.parametrize("bits", [0, 4])
@pytest.mark.parametrize("ahead", [True, False], ids=["sealed_ahead", "on_demand"])
def test_merged_layer_launch(bits, ahead):
    """merge_groups: a 41-block layer in 16-block causal groups goes to the
    device as one launch (one layer group around the groups' swaps, K1 V1 K2
    V2 K3 V3; sealed ahead it is one layer prefetch and one DMA).  Each layer
    spends exactly 2 x 41 tickets, every swap is served by the prefetch when
    sealed ahead, and the caches end bit-exact (bf16), or equal to the oracle
    codec's decode of the packets (int4).  The order the tickets follow is
    pinned on the CPU by the host runtime's sanitizer stress test, which logs
    every record's AAD."""
    rng = np.random.default_rng(150 + bits + int(ahead))
    heads, dim, ncpu, nslots, nlayers = 2, 128, 41, 64, 3
    shape = si.LayerShape(heads, dim, bits)
    sess = si.GcmSession(KEY, SALT, 10 + bits, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        if bits:
            layers = _codec_layers(rng, nlayers, ncpu, heads, dim, bits)
            host_layers = [packets for packets, _ in layers]
        else:
            host_layers = _layers(rng, nlayers, ncpu, heads, dim)
        nt = si.NativeTransfer(sess, shape, causal_group_blocks=16, pipeline_seal=ahead, merge_groups=True)
        slot_ids = rng.permutation(nslots)[:ncpu]
        mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
        before = si.transfer_prefetch_stats()
        caches_l = [caches(nslots, heads, dim) for _ in range(nlayers)]
        for layer in range(nlayers):
            t0 = si.new_transfer_ticket()
            nt.single_layer_kv_transfer((host_layers[layer], mapping), caches_l[layer])
            assert si.new_transfer_ticket() == t0 + 2 * ncpu + 1
        after = si.transfer_prefetch_stats()
        served = (after["ready"] - before["ready"]) + (after["busy_fallback"] - before["busy_fallback"])
        missing = after["missing_fallback"] - before["missing_fallback"]
        assert (served, missing) == ((nlayers * 6, 0) if ahead else (0, nlayers * 6))
        assert int(_lib.load().secure_infer_count_ready_unconsumed_gcm_tickets()) == 0
        idx = torch.from_numpy(slot_ids.astype(np.int64)).to(DEV)
        for layer in range(nlayers):
            assert nt.wait_layer(layer) == 0
            ck, cv = caches_l[layer]
            got = [ck.index_select(0, idx).cpu().numpy(), cv.index_select(0, idx).cpu().numpy()]
            for k in range(2):
                if bits:
                    packets = host_layers[layer][k].numpy()
                    for i in range(ncpu):
                        assert np.array_equal(got[k][i].view(np.uint16),
                                              O.codec_decode(packets[i], heads, dim, bits, k)), (layer, k, i)
                else:
                    assert np.array_equal(got[k], host_layers[layer][k].numpy()), (layer, k)
            untouched = np.setdiff1d(np.arange(nslots), slot_ids)
            assert (host(ck)[untouched].view(np.uint8) == 0x3C).all()
    finally:
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


@pytest.mark.parametrize("shots", [1, 2], ids=["repaired", "final"])
def test_merged_layer_tamper(shots):
    """A V record of the middle causal group of a merged, sealed-ahead layer
    corrupted once is re-sealed by the strict retry and the layer
    authenticates; corrupted twice, the layer fails, that slot reads as
    zeros, and every other slot is still bit-exact."""
    rng = np.random.default_rng(160 + shots)
    heads, dim, ncpu, nslots, layer = 2, 128, 41, 48, 0
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 20 + shots, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        (hk, hv), = _layers(rng, 1, ncpu, heads, dim)
        slot_ids = rng.permutation(nslots)[:ncpu]
        mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
        victim = 17  # in the group [9, 25)
        si.inject_h2d_tamper(layer=layer, kind=1, host_block=victim, shots=shots)
        nt = si.NativeTransfer(sess, shape, causal_group_blocks=16, merge_groups=True)
        ck, cv = caches(nslots, heads, dim)
        nt.single_layer_kv_transfer(((hk, hv), mapping), (ck, cv))
        assert nt.wait_layer(layer) == (0 if shots == 1 else -1)
        kk, vv = host(ck), host(cv)
        for c, sl in enumerate(slot_ids):
            assert np.array_equal(kk[sl], hk[c].numpy())
            if shots == 2 and c == victim:
                assert (vv[sl] == 0).all()
            else:
                assert np.array_equal(vv[sl], hv[c].numpy()), c
    finally:
        si.inject_h2d_tamper(shots=0)
        si.retire_transfer_prefetches()
        si.clear_host_ranges()


def test_job_authentication_spans_layers():
    """secure_infer_recovery_wait_job_authentication (secure_infer.cpp:7336-7372):
    every record of the job on every layer, no retry; 1 / 0 / -1."""
    rng = np.random.default_rng(143)
    heads, dim, ncpu, nslots = 2, 128, 6, 12
    shape = si.LayerShape(heads, dim)
    sess = si.GcmSession(KEY, SALT, 4, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        host_layers = _layers(rng, 2, ncpu, heads, dim)
        mapping = torch.tensor([[1, 3], [4, 0], [5, 7]], dtype=torch.int64)
        nt = si.NativeTransfer(sess, shape)
        si.set_job_id(7001)
        for layer in range(2):
            nt.single_layer_kv_transfer((host_layers[layer], mapping), caches(nslots, heads, dim))
        assert si.wait_job_authentication(7001) == 1
        si.set_job_id(7002)
        si.inject_h2d_tamper(layer=1, kind=0, host_block=4, shots=1)
        nt.layer = 0
        for layer in range(2):
            nt.single_layer_kv_transfer((host_layers[layer], mapping), caches(nslots, heads, dim))
        assert si.wait_job_authentication(7002) == 0   # no strict retry on the job path
        assert si.wait_job_authentication(7003) == -1  # no records
    finally:
        si.inject_h2d_tamper(shots=0)
        si.set_job_id(0)
        si.clear_host_ranges()


LEDGER_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import secure_infer_amd as si
heads, dim = 2, 128
shape = si.LayerShape(heads, dim)
sess = si.GcmSession(bytes(16), b"abcd", 0, max_record_bytes=shape.record_bytes)
hk = torch.zeros((8, 128, heads, dim), dtype=torch.int16)
hv = torch.ones((8, 128, heads, dim), dtype=torch.int16)
ck = torch.zeros((8, 128, heads, dim), dtype=torch.int16, device="cuda")
cv = torch.zeros_like(ck)
nt = si.NativeTransfer(sess, shape, pipeline_seal=False)
m = torch.tensor([[0, 1], [2, 3], [7, 5]], dtype=torch.int64)
assert nt.prefetch_kv_transfer(((hk, hv), m), 0)
nt.single_layer_kv_transfer(((hk, hv), m), (ck, cv))
nt.single_layer_kv_transfer(((hk, hv), m), (ck, cv))
assert nt.wait_layer(0) == 0 and nt.wait_layer(1) == 0
si.drain_h2d_profile_after_job()
print("done")
"""


MERGED_LEDGER_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import secure_infer_amd as si
heads, dim, n = 2, 128, 41
shape = si.LayerShape(heads, dim)
sess = si.GcmSession(bytes(16), b"abcd", 0, max_record_bytes=shape.record_bytes)
hk = torch.zeros((n, 128, heads, dim), dtype=torch.int16)
hv = torch.ones((n, 128, heads, dim), dtype=torch.int16)
ck = torch.zeros((64, 128, heads, dim), dtype=torch.int16, device="cuda")
cv = torch.zeros_like(ck)
m = torch.stack((torch.arange(n), torch.arange(n) + 20), 1).to(torch.int64).contiguous()
ahead = si.NativeTransfer(sess, shape, causal_group_blocks=16, merge_groups=True)
ahead.single_layer_kv_transfer(((hk, hv), m), (ck, cv))
late = si.NativeTransfer(sess, shape, causal_group_blocks=16, merge_groups=True, pipeline_seal=False)
late.layer = 1
late.single_layer_kv_transfer(((hk, hv), m), (ck, cv))
assert ahead.wait_layer(0) == 0 and late.wait_layer(1) == 0
assert torch.equal(cv[20:20 + n].cpu(), hv) and torch.equal(ck[20:20 + n].cpu(), hk)
si.drain_h2d_profile_after_job()
print("done")
"""


def test_merged_layer_is_one_launch(tmp_path):
    """With merge_groups a 41-block layer in three causal groups is one row
    of the H2D ledger (one launch of 82 records), sealed ahead or on demand."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    csv = tmp_path / "h2d.csv"
    env = dict(os.environ, SECURE_INFER_H2D_PROFILE=str(csv))
    out = subprocess.run([sys.executable, "-c", MERGED_LEDGER_SCRIPT, str(Path(__file__).resolve().parent.parent)],
                         env=env, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0 and "done" in out.stdout, out.stderr[-2000:]
    rows = [l.split(",") for l in csv.read_text().strip().splitlines()[1:]]
    src = sorted((r[0], r[1], r[2], r[4].replace("prefetch_waited", "prefetched")) for r in rows)
    assert src == [("0", "2", "82", "prefetched"), ("1", "2", "82", "sealed")]


def test_h2d_profile_ledger(tmp_path):
    """SECURE_INFER_H2D_PROFILE: one CSV row per launch with host seal, H2D copy
    and kernel time (the reference's per-copy rows, secure_infer.cpp:6085-6137);
    a layer group's K and V swaps go out as one launch (kind 2)."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    csv = tmp_path / "h2d.csv"
    env = dict(os.environ, SECURE_INFER_H2D_PROFILE=str(csv))
    out = subprocess.run([sys.executable, "-c", LEDGER_SCRIPT, str(Path(__file__).resolve().parent.parent)],
                         env=env, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0 and "done" in out.stdout, out.stderr[-2000:]
    lines = csv.read_text().strip().splitlines()
    assert lines[0] == "layer,kind,records,record_bytes,source,seal_us,h2d_copy_us,kernel_us"
    rows = [l.split(",") for l in lines[1:]]
    assert len(rows) == 2
    # layer 0 was sealed ahead of demand (ready or still sealing when its swap
    # came), layer 1 on demand
    src = sorted((r[0], r[1], r[4].replace("prefetch_waited", "prefetched")) for r in rows)
    assert src == [("0", "2", "prefetched"), ("1", "2", "sealed")]
    for r in rows:
        assert int(r[2]) == 6 and int(r[3]) == 128 * 2 * 128 * 2
        assert float(r[5]) > 0 and float(r[6]) > 0 and float(r[7]) > 0


def test_h2d_profile_ledger_records(tmp_path):
    """SECURE_INFER_H2D_PROFILE_RECORDS=1: one row per record in the
    reference's per-copy column set (secure_infer.cpp:1846-1847, 5649-5690):
    'H2D', payload and wire bytes, the record's own seal time, the enqueue
    times and device phases of the launch that carried it, and whether it
    was sealed ahead of demand (cpu_prediction_hit)."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    csv = tmp_path / "h2d_records.csv"
    env = dict(os.environ, SECURE_INFER_H2D_PROFILE=str(csv), SECURE_INFER_H2D_PROFILE_RECORDS="1")
    out = subprocess.run([sys.executable, "-c", LEDGER_SCRIPT, str(Path(__file__).resolve().parent.parent)],
                         env=env, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0 and "done" in out.stdout, out.stderr[-2000:]
    lines = csv.read_text().strip().splitlines()
    assert lines[0] == ("direction,bytes,aligned_bytes,total_us,cpu_crypto_us,device_pipeline_us,host_wait_us,"
                        "copy_enqueue_us,kernel_enqueue_us,h2d_device_us,kernel_execute_us,d2d_device_us,"
                        "device_total_us,device_timing_valid,crypto_mode,cpu_prediction_hit")
    rows = [[int(x) if x.isdigit() else x for x in l.split(",")] for l in lines[1:]]
    nbytes = 128 * 2 * 128 * 2
    assert len(rows) == 12  # two layers of 3 K and 3 V records
    for r in rows:
        assert r[0] == "H2D" and r[1] == nbytes and r[2] == si.wire_stride(nbytes)
        assert r[13] == 1 and r[14] == 0 and r[6] == 0 and r[11] == 0
        assert r[4] > 0 and r[9] > 0 and r[10] > 0 and r[12] >= r[10] and r[5] == r[12]
        assert r[3] >= r[4] + r[12] - 1  # rounding of the summed parts
    # layer 0 was sealed ahead of demand, layer 1 on demand
    assert sorted(r[15] for r in rows) == [0] * 6 + [1] * 6


@pytest.mark.parametrize("shots", [1, 2], ids=["repaired", "final"])
def test_codec_auth_wait(shots):
    """NativeTransfer(codec_auth_wait=True) over an int4 layer whose V record
    is corrupted once: the strict retry re-seals it and the transfer returns
    with every slot bit-exact.  Corrupted twice: the transfer raises 'Packed
    KV authentication failed' (the reference's assert before decode_into,
    transport_codec.py:168-174) and that record's slot reads as zeros, every
    other slot bit-exact."""
    rng = np.random.default_rng(170 + shots)
    heads, dim, ncpu, nslots, layer, bits = 2, 128, 20, 32, 0, 4
    shape = si.LayerShape(heads, dim, bits)
    sess = si.GcmSession(KEY, SALT, 30 + shots, max_record_bytes=shape.record_bytes)
    si.clear_host_ranges()
    try:
        (packets, _), = _codec_layers(rng, 1, ncpu, heads, dim, bits)
        slot_ids = rng.permutation(nslots)[:ncpu]
        mapping = torch.from_numpy(np.stack([np.arange(ncpu), slot_ids], 1).astype(np.int64))
        victim = 7
        si.inject_h2d_tamper(layer=layer, kind=1, host_block=victim, shots=shots)
        nt = si.NativeTransfer(sess, shape, causal_group_blocks=16, codec_auth_wait=True)
        ck, cv = caches(nslots, heads, dim)
        if shots == 1:
            nt.single_layer_kv_transfer((packets, mapping), (ck, cv))
        else:
            with pytest.raises(RuntimeError, match="Packed KV authentication failed"):
                nt.single_layer_kv_transfer((packets, mapping), (ck, cv))
        assert nt.layer == layer + 1
        kk, vv = host(ck), host(cv)
        for c, sl in enumerate(slot_ids):
            assert np.array_equal(kk[sl].view(np.uint16), O.codec_decode(packets[0][c].numpy(), heads, dim, bits, 0))
            if shots == 2 and c == victim:
                assert (vv[sl] == 0).all()
            else:
                assert np.array_equal(vv[sl].view(np.uint16),
                                      O.codec_decode(packets[1][c].numpy(), heads, dim, bits, 1)), c
    finally:
        si.inject_h2d_tamper(shots=0)
        si.retire_transfer_prefetches()
        si.clear_host_ranges()
