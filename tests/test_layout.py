"""The host's share layout of a layer launch, checked on the CPU.

A layer launch cuts the records' GHASH input into rows of 256 blocks and gives
each workgroup of the record kernel one contiguous share of the records'
concatenated rows (`secure_infer_gpu_layout` returns the layout the launch
would use; no device call).  The kernel relies on these properties, checked
here over seeded shapes, CU counts and tuning values:

* the shares tile [0, nrec * R) in order, R = the least number of rows that
  holds a record's AAD and payload blocks;
* no share is longer than R rows, so a share has one or two segments (the end
  of one record, the start of the next);
* a share that straddles two records gains rows after paying the straddle
  cost: its rows plus the cost fit in the longest share;
* with pairs, workgroup w takes the whole records 2w and 2w + 1;
* there are at least as many workgroups as records unless pairs are laid out,
  whole rounds of one per CU when the records outnumber the CUs;
* an equal split (too many workgroups to lay out one by one) gives each
  workgroup at most R rows;
* the tag-mask flag is set exactly when a record's first row holds a
  ciphertext block after its last AAD block.
"""
import ctypes as ct

import numpy as np
import pytest

import secure_infer_amd as si
from secure_infer_amd import _lib

T = 256
MAX_WG = 768


@pytest.fixture
def lib():
    L = _lib.load()
    assert L.secure_infer_gpu_set_chunk_rows(si.gcm.DEFAULT_CHUNK_ROWS) == 0
    assert L.secure_infer_gpu_set_straddle_rows(si.gcm.DEFAULT_STRADDLE_ROWS) == 0
    yield L
    assert L.secure_infer_gpu_set_chunk_rows(si.gcm.DEFAULT_CHUNK_ROWS) == 0
    assert L.secure_infer_gpu_set_straddle_rows(si.gcm.DEFAULT_STRADDLE_ROWS) == 0


def _layout(L, nrec, nbytes, aad, cus):
    info = (ct.c_uint32 * 5)()
    starts = (ct.c_uint32 * (MAX_WG + 1))()
    assert L.secure_infer_gpu_layout(nrec, nbytes, aad, cus, info, starts, MAX_WG + 1) == 0
    W, R, use, pairs, ek = (int(x) for x in info)
    return W, R, use, pairs, ek, ([int(x) for x in starts[:W + 1]] if use else None)


def _check(L, nrec, nbytes, aad, cus, min_rows, straddle):
    W, R, use, pairs, ek, starts = _layout(L, nrec, nbytes, aad, cus)
    case = (nrec, nbytes, aad, cus, min_rows, straddle)
    a, n = -(-aad // 16), -(-nbytes // 16)
    assert (R - 1) * T < a + n <= R * T, case
    pad = R * T - (a + n)
    assert ek == int(a >= 1 and n >= 1 and pad + a <= T - 1), case
    G = nrec * R
    if pairs:
        assert use == 1 and nrec > cus and W == (nrec + 1) // 2, case
        assert starts == [min(2 * w, nrec) * R for w in range(W + 1)], case
        return
    assert W >= nrec, case
    if nrec > cus:
        assert W % cus == 0 or W == G, case
    if not use:
        assert W > MAX_WG and -(-G // W) <= R, case
        return
    assert starts[0] == 0 and starts[-1] == G, case
    lens = np.diff(np.array(starts, dtype=np.int64))
    assert (lens >= 0).all() and lens.max() <= R, case
    longest = int(lens.max())
    for g0, g1 in zip(starts[:-1], starts[1:]):
        if g1 == g0:
            continue
        r0 = g0 // R
        if g1 > (r0 + 1) * R:  # straddles records r0 and r0 + 1
            assert g1 - g0 + straddle <= longest, case
            assert g1 <= (r0 + 2) * R, case


def test_layout_refuses_bad_arguments(lib):
    info = (ct.c_uint32 * 5)()
    starts = (ct.c_uint32 * 4)()
    assert lib.secure_infer_gpu_layout(0, 4096, 64, 256, info, starts, 4) == -1
    assert lib.secure_infer_gpu_layout(4, 0, 64, 256, info, starts, 4) == -1
    assert lib.secure_infer_gpu_layout(4, 4096, 64, 0, info, starts, 4) == -1
    assert lib.secure_infer_gpu_layout(4, 4096, 64, MAX_WG + 1, info, starts, 4) == -1
    assert lib.secure_infer_gpu_layout(4, 4096, 64, 256, None, starts, 4) == -1
    # four one-row records on 256 CUs: four shares, five boundaries needed
    assert lib.secure_infer_gpu_layout(4, 4096, 64, 256, info, starts, 4) == -1


def test_layout_of_the_benchmark_layers(lib):
    """The bf16 Llama-3-8B layer (96 records of 256 KiB) under the default
    tuning: 26-row shares on all 256 CUs, 64 of them straddling; the 70B
    writeback layer (512 int4 packets of 81,936 B): pairs of whole records."""
    W, R, use, pairs, ek, starts = _layout(lib, 96, 262144, 64, 256)
    assert (W, R, use, pairs, ek) == (256, 65, 1, 0, 0)
    lens = np.diff(starts)
    straddling = sum(1 for g0, g1 in zip(starts[:-1], starts[1:]) if g1 > (g0 // R + 1) * R)
    assert lens.max() == 26 and straddling == 64
    W, R, use, pairs, ek, starts = _layout(lib, 512, 81936, 64, 256)
    assert (W, R, pairs) == (256, 21, 1)


def test_layout_invariants_over_random_shapes(lib):
    rng = np.random.default_rng(2024)
    for _ in range(3000):
        nrec = int(rng.choice([1, 2, 3, int(rng.integers(1, 300)), int(rng.integers(1, 3000))]))
        nbytes = int(rng.choice([int(rng.integers(1, 4097)), int(rng.integers(1, 1 << 18)),
                                 int(rng.integers(1, 1 << 21))]))
        aad = int(rng.choice([0, 16, 64, 100]))
        cus = int(rng.choice([1, 7, 80, 256, 304, MAX_WG]))
        min_rows = int(rng.choice([1, 2, 3, 5, 8, 16, 64, 256]))
        straddle = int(rng.choice([0, 1, 2, 6, 13, 256]))
        assert lib.secure_infer_gpu_set_chunk_rows(min_rows) == 0
        assert lib.secure_infer_gpu_set_straddle_rows(straddle) == 0
        _check(lib, nrec, nbytes, aad, cus, min_rows, straddle)


def test_layout_knobs_take_effect(lib):
    """A straddle cost above every share length stops straddling; the minimum
    rows per share bounds the number of workgroups."""
    assert lib.secure_infer_gpu_set_straddle_rows(256) == 0
    W, R, use, pairs, ek, starts = _layout(lib, 96, 262144, 64, 256)
    assert all(g1 <= (g0 // R + 1) * R for g0, g1 in zip(starts[:-1], starts[1:]) if g1 > g0)
    assert lib.secure_infer_gpu_set_straddle_rows(si.gcm.DEFAULT_STRADDLE_ROWS) == 0
    assert lib.secure_infer_gpu_set_chunk_rows(64) == 0
    W, R, use, pairs, ek, starts = _layout(lib, 4, 262144, 64, 256)
    assert W == -(-4 * R // 64) and np.diff(starts).max() <= R
