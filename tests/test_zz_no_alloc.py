"""The allocation-free reload (secure_infer_gpu_reload_layer_noalloc) against
secure_infer_gpu_reload_layer on the same records, through the C-ABI: two
calls in a row per case, the second with fewer records, each checked for
identical cache contents, record statuses and fail counts (bit-exact), and
against the oracle.  Cases cover the codec staging (int8 with a tampered
record, int4) and the pair layout's parking area (more records than CUs).
Requests beyond the scratch limits, or that bring their own staging, are
refused with -1 before any work."""
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


def reload(entry, sess, wire, n, nb, caches, slots, t0, bits, heads, dim, layer, staging, fail):
    d = _lib.SiReloadDesc(
        wire=wire.data_ptr(), wire_stride=W.stride(n), bytes=n, nrec=2 * nb, n_k=nb, iv_words=None,
        ticket_base=t0, cache_k=caches[0].data_ptr(), cache_v=caches[1].data_ptr(),
        slot_bytes=caches[0][0].numel() * 2, nslots=caches[0].shape[0], slots=slots.data_ptr(),
        codec_bits=bits, heads=heads, head_dim=dim, layer=layer,
        staging=None if staging is None else staging.data_ptr(), fail_count=fail.data_ptr())
    fn = getattr(_lib.load(), entry)
    return fn(ct.c_void_p(torch.cuda.current_stream().cuda_stream), sess._h, ct.byref(d))


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
