"""The allocation-free reload (secure_infer_gpu_reload_layer_noalloc) against
secure_infer_gpu_reload_layer on the same records, through the C-ABI: two
calls in a row per case, the second with fewer records, each checked for
identical cache contents, record statuses and fail counts (bit-exact), and
against the oracle.  Cases cover the codec staging (int8 with a tampered
record, int4) and the pair layout's parking area (more records than CUs).
Requests beyond the scratch limits, or that bring their own staging, are
refused with -1 before any work.

Calls share one scratch array per GPU and take it for themselves on the
device; a call that finds it taken fails every record closed.  Tested with
the scratch held by the test hook (every record status 0, zeroed, counted),
with two calls in flight on two streams at once (each either verifies
exactly or fails closed entirely, never a mix) and with a serial call after
both (verifies)."""
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
KEY = bytes(range(0x90, 0xA0))
SALT = b"\x01\x02\x03\x05"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def make_layer(rng, bits, heads, dim, nb, layer, t0, tamper=()):
    kinds = [0] * nb + [1] * nb
    blocks = W.bf16_blocks(rng, 2 * nb, heads, dim)
    if bits:
        payloads = [O.codec_encode(blocks[r], bits, kinds[r], layer) for r in range(2 * nb)]
    else:
        payloads = [blocks[r].view(np.uint8).reshape(-1) for r in range(2 * nb)]
    n = payloads[0].size
    wire = W.build_wire(KEY, SALT, payloads, kinds, layer, list(range(nb)) * 2, t0)
    for r in tamper:
        wire[r * W.stride(n) + 5] ^= 0x11
    if bits:
        want = np.stack([O.codec_decode(payloads[r], heads, dim, bits, kinds[r]) for r in range(2 * nb)])
    else:
        want = blocks.copy()
    want[list(tamper)] = 0
    return wire, n, want


def reload(entry, sess, wire, n, nb, caches, slots, t0, bits, heads, dim, layer, staging, fail, stream=None):
    d = _lib.SiReloadDesc(
        wire=wire.data_ptr(), wire_stride=W.stride(n), bytes=n, nrec=2 * nb, n_k=nb, iv_words=None,
        ticket_base=t0, cache_k=caches[0].data_ptr(), cache_v=caches[1].data_ptr(),
        slot_bytes=caches[0][0].numel() * 2, nslots=caches[0].shape[0], slots=slots.data_ptr(),
        codec_bits=bits, heads=heads, head_dim=dim, layer=layer,
        staging=None if staging is None else staging.data_ptr(), fail_count=fail.data_ptr())
    fn = getattr(_lib.load(), entry)
    st = stream if stream is not None else torch.cuda.current_stream()
    return fn(ct.c_void_p(st.cuda_stream), sess._h, ct.byref(d))


def statuses(dw, nrec, n):
    st = dw.cpu().numpy().reshape(nrec, W.stride(n))
    return st[:, W.align32(n) + 16:W.align32(n) + 20].copy().view("<u4").ravel()


class Call:
    """One allocation-free reload of a fresh layer into its own caches."""

    def __init__(self, rng, bits, heads, dim, nb, layer, t0, tamper, nslots=64):
        self.nb, self.bits, self.heads, self.dim, self.layer, self.t0 = nb, bits, heads, dim, layer, t0
        self.tamper = tamper
        wire, self.n, self.want = make_layer(rng, bits, heads, dim, nb, layer, t0, tamper)
        self.sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=self.n)
        self.slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
        self.slots = dev(np.concatenate([self.slot_ids, self.slot_ids]))
        self.caches = [torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV) for _ in range(2)]
        for c in self.caches:
            c.view(torch.uint8).fill_(0x3C)
        self.dw = dev(wire)
        self.fail = torch.zeros(1, dtype=torch.int32, device=DEV)

    def launch(self, stream=None):
        if stream is not None:
            stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the current stream
        return reload("secure_infer_gpu_reload_layer_noalloc", self.sess, self.dw, self.n, self.nb, self.caches,
                      self.slots, self.t0, self.bits, self.heads, self.dim, self.layer, None, self.fail, stream)

    def outcome(self):
        """'verified' or 'failed_closed'; asserts the result is exactly one of them."""
        torch.cuda.synchronize()
        nrec = 2 * self.nb
        st = statuses(self.dw, nrec, self.n)
        fail = int(self.fail.item())
        idx = dev(self.slot_ids)
        got = [self.caches[k].index_select(0, idx) for k in range(2)]
        mask = torch.ones(self.caches[0].shape[0], dtype=torch.bool, device=DEV)
        mask[idx] = False
        for c in self.caches:  # slots outside the mapping are never touched
            assert bool((c[mask].view(torch.uint8) == 0x3C).all())
        want_st = np.ones(nrec, np.uint32)
        want_st[list(self.tamper)] = 0
        if np.array_equal(st, want_st):
            assert fail == len(self.tamper)
            want = dev(self.want.view(np.int16))
            assert torch.equal(got[0], want[:self.nb]) and torch.equal(got[1], want[self.nb:])
            return "verified"
        assert not st.any(), f"statuses mix verified and refused records: {st}"
        assert fail == nrec, f"fail count {fail} for {nrec} refused records"
        assert not bool(got[0].any()) and not bool(got[1].any()), "a refused record kept data"
        return "failed_closed"


@pytest.mark.parametrize("bits,heads,dim,calls", [
    (8, 4, 128, [(8, (3,)), (3, ())]),           # int8, staging; tampered K record 3 first
    (4, 4, 128, [(64, (70,)), (5, ())]),         # int4 Qwen-size layer, then a small one
    (0, 1, 64, [(160, (1, 200)), (7, ())]),      # 320 records > CUs: pairs and their parking area
], ids=["int8", "int4", "bf16_pairs"])
def test_noalloc_reload_matches_reload_layer(bits, heads, dim, calls):
    rng = np.random.default_rng(4242 + bits)
    layer, nslots = 3, 512
    for call, (nb, tamper) in enumerate(calls):
        t0 = 100000 * (call + 1) + bits
        wire, n, want = make_layer(rng, bits, heads, dim, nb, layer, t0, tamper)
        sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
        slot_ids = rng.permutation(nslots)[:nb].astype(np.int64)
        slots = dev(np.concatenate([slot_ids, slot_ids]))
        outs = []
        for entry in ("secure_infer_gpu_reload_layer", "secure_infer_gpu_reload_layer_noalloc"):
            caches = [torch.zeros((nslots, 128, heads, dim), dtype=torch.int16, device=DEV) for _ in range(2)]
            for c in caches:
                c.view(torch.uint8).fill_(0x3C)
            dw = dev(wire)
            fail = torch.zeros(1, dtype=torch.int32, device=DEV)
            staging = None
            if bits and entry == "secure_infer_gpu_reload_layer":
                staging = torch.empty(2 * nb * W.align32(n), dtype=torch.uint8, device=DEV)
            assert reload(entry, sess, dw, n, nb, caches, slots, t0, bits, heads, dim, layer, staging, fail) == 0
            torch.cuda.synchronize()
            st = dw.cpu().numpy().reshape(2 * nb, W.stride(n))[:, W.align32(n) + 16:W.align32(n) + 20]
            outs.append((caches, st.copy(), int(fail.item())))
        (ca, sa, fa), (cb, sb, fb) = outs
        assert torch.equal(ca[0], cb[0]) and torch.equal(ca[1], cb[1]), f"call {call}: caches differ"
        assert np.array_equal(sa, sb) and fa == fb == len(tamper)
        want_dev = dev(want.view(np.int16))
        idx = dev(slot_ids)
        assert torch.equal(cb[0].index_select(0, idx), want_dev[:nb])
        assert torch.equal(cb[1].index_select(0, idx), want_dev[nb:])


def test_noalloc_refuses_requests_beyond_its_scratch():
    heads, dim, bits, nb = 8, 128, 8, 256          # 512 int8 packets: 75.5 MB of staging > 64 MiB
    n = si.codec_width(bits, heads, dim)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=n)
    wire = torch.zeros(1024, dtype=torch.uint8, device=DEV)
    caches = [torch.zeros((2, 128, heads, dim), dtype=torch.int16, device=DEV) for _ in range(2)]
    slots = torch.zeros(2 * nb, dtype=torch.int64, device=DEV)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert reload("secure_infer_gpu_reload_layer_noalloc", sess, wire, n, nb, caches, slots, 1, bits, heads,
                  dim, 0, None, fail) == -1
    # a caller-provided staging buffer is refused too
    staging = torch.zeros(16, dtype=torch.uint8, device=DEV)
    assert reload("secure_infer_gpu_reload_layer_noalloc", sess, wire, n, 1, caches, slots[:2], 1, bits, heads,
                  dim, 0, staging, fail) == -1
    torch.cuda.synchronize()
    assert int(fail.item()) == 0 and not bool(caches[0].any())


@pytest.mark.parametrize("bits", [0, 4], ids=["bf16", "int4"])
def test_noalloc_taken_scratch_fails_closed_then_recovers(bits):
    """While the scratch is held (the test hook's token), a call must not
    touch it: every record fails closed and is counted.  Once released, the
    next call verifies (a held owner word never sticks to a later call)."""
    rng = np.random.default_rng(5150 + bits)
    L = _lib.load()
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    held = Call(rng, bits, 4, 128, 5, 2, 7000 + bits, (1,))
    assert L.secure_infer_test_noalloc_hold(stream, 1) == 0
    try:
        assert held.launch() == 0
        assert held.outcome() == "failed_closed"
    finally:
        assert L.secure_infer_test_noalloc_hold(stream, 0) == 0
    after = Call(rng, bits, 4, 128, 5, 2, 7100 + bits, (1, 7))
    assert after.launch() == 0
    assert after.outcome() == "verified"


def test_noalloc_overlapping_calls_never_mix():
    """Two calls in flight at once on two streams, over disjoint caches and
    each with a tampered record: each either verifies exactly (statuses,
    fail count, slots) or fails closed entirely; a serial call after them
    verifies."""
    rng = np.random.default_rng(5252)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    seen = []
    for rnd in range(4):
        a = Call(rng, 4, 4, 128, 32, 1, 20000 + 1000 * rnd, (3,))
        b = Call(rng, 0, 2, 128, 24, 2, 40000 + 1000 * rnd, (30,))
        torch.cuda.synchronize()
        assert a.launch(s1) == 0
        assert b.launch(s2) == 0
        seen += [a.outcome(), b.outcome()]
    print("overlap outcomes:", seen, flush=True)
    last = Call(rng, 8, 4, 128, 8, 3, 90000, (0,))
    assert last.launch() == 0
    assert last.outcome() == "verified"
