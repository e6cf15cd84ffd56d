"""GPU parity sweep over layer shapes: the host's share layout of a layer
(shares of rows per workgroup, straddling shares, rounds and pairs of whole
records when the records outnumber the CUs) for record counts around one and
two per CU and record sizes with partial last blocks.

Every reload is checked record by record against OpenSSL-sealed records
(statuses, fail count, slot bytes, untouched slots); every writeback's
ciphertext and tags against OpenSSL over the gathered slot bytes.  The
shapes are run twice in one thread, interleaved, so a layout reused from the
library's per-thread layout cache must be the one of the current shape.  A
seeded random sweep adds shapes and layout knobs (minimum rows per share,
straddle cost) that no fixed list names.
Byte and integer work: all comparisons are bit-exact.
"""
import functools

import numpy as np
import pytest
import torch

import secure_infer_amd as si
from tests import wire as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
KEY = bytes(range(0x40, 0x50))
SALT = b"\x5a\xa5\x0f\xf0"
FILL = 0x3C

# (records, record bytes): one record; fewer records than CUs; a partial
# round; exactly one and two records per CU; more records than CUs (rounds or
# pairs of whole records); records of many rows whose shares straddle.
SHAPES = [(1, 4001), (3, 16384), (255, 4000), (256, 4096), (257, 4080), (512, 2000),
          (513, 4096), (700, 1000), (96, 65535)]


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _reload_case(sess, rng, nrec, n, ticket0, strict=False):
    n_k = nrec // 2
    kinds = [0] * n_k + [1] * (nrec - n_k)
    payloads = [rng.integers(0, 256, n, dtype=np.uint8) for _ in range(nrec)]
    wire = W.build_wire(KEY, SALT, payloads, kinds, 3, list(range(nrec)), ticket0)
    st = W.stride(n)
    bad = set(rng.choice(nrec, size=min(3, nrec), replace=False).tolist()) if nrec > 1 else {0}
    for r in bad:
        wire[r * st + int(rng.integers(0, n))] ^= 0x01
    nslots = nrec + 8
    slot_bytes = (n + 15) // 16 * 16 + 32
    slots_np = np.empty(nrec, np.int64)
    slots_np[:n_k] = rng.permutation(nslots)[:n_k]
    slots_np[n_k:] = rng.permutation(nslots)[:nrec - n_k]
    ck = torch.full((nslots, slot_bytes), FILL, dtype=torch.uint8, device=DEV)
    cv = torch.full_like(ck, FILL)
    fail = torch.zeros(1, dtype=torch.int32, device=DEV)
    dw = _dev(wire)
    sess.reload_layer(dw, n, nrec, n_k, ck, cv, _dev(slots_np), ticket_base=ticket0, fail_count=fail,
                      verify_before_release=strict)
    kk, vv, ww = _host(ck), _host(cv), _host(dw)
    toff = W.align32(n)
    statuses = [int(ww[r * st + toff + 16:r * st + toff + 20].view(np.uint32)[0]) for r in range(nrec)]
    assert statuses == [0 if r in bad else 1 for r in range(nrec)], (nrec, n)
    assert int(_host(fail)[0]) == len(bad), (nrec, n)
    for r in range(nrec):
        row = (kk if r < n_k else vv)[slots_np[r]]
        if r in bad:
            assert not row[:n].any(), (nrec, n, r)
        else:
            assert np.array_equal(row[:n], payloads[r]), (nrec, n, r)
    for cache, used in ((kk, slots_np[:n_k]), (vv, slots_np[n_k:])):
        untouched = np.setdiff1d(np.arange(nslots), used)
        assert np.all(cache[untouched] == FILL), (nrec, n)


def _writeback_case(sess, rng, nrec, n, ticket0):
    n_k = nrec - nrec // 2
    kinds = [0] * n_k + [1] * (nrec - n_k)
    nslots = nrec + 5
    slot_bytes = (n + 15) // 16 * 16
    data = rng.integers(0, 256, (2, nslots, slot_bytes), dtype=np.uint8)
    ck, cv = _dev(data[0]), _dev(data[1])
    slots_np = np.concatenate([rng.permutation(nslots)[:n_k],
                               rng.permutation(nslots)[:nrec - n_k]]).astype(np.int64)
    plain = [data[kinds[r]][slots_np[r]][:n] for r in range(nrec)]
    wire = W.wire_aads(KEY, SALT, n, kinds, 6, list(range(nrec)), ticket0)
    dw = _dev(wire)
    sess.writeback_layer(dw, n, nrec, n_k, ck, cv, _dev(slots_np), ticket_base=ticket0)
    ww = _host(dw)
    expect = W.build_wire(KEY, SALT, plain, kinds, 6, list(range(nrec)), ticket0, direction=2)
    st, toff = W.stride(n), W.align32(n)
    for r in range(nrec):
        o = r * st
        assert np.array_equal(ww[o:o + n], expect[o:o + n]), (nrec, n, r, "ciphertext")
        assert np.array_equal(ww[o + toff:o + toff + 16], expect[o + toff:o + toff + 16]), (nrec, n, r, "tag")


@pytest.mark.parametrize("direction", ["reload", "writeback"])
def test_layout_sweep_matches_openssl(direction):
    rng = np.random.default_rng(7100 if direction == "reload" else 7200)
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=max(n for _, n in SHAPES))
    case = _reload_case if direction == "reload" else _writeback_case
    ticket = 1
    for rep in range(2):
        order = SHAPES if rep == 0 else SHAPES[::-1]
        for nrec, n in order:
            print(f"{direction} rep {rep}: {nrec} records x {n} B", flush=True)
            case(sess, rng, nrec, n, ticket)
            ticket += nrec


@pytest.mark.parametrize("direction", ["reload", "reload_verify_first", "writeback"])
def test_random_layouts_match_openssl(direction):
    """Seeded random shapes and layout knobs beyond the hand-picked ones:
    record counts from one to past four per CU, record sizes from one byte
    to past four rows (most with a partial last block), the minimum rows per
    share (1 to 8) and the straddle cost (0 to 13), so shares straddle, pair
    up or run in rounds in combinations no fixed list names.  Each case
    against OpenSSL as above; reloads also with verify-before-release (tags
    first, then decryption released by status)."""
    rng = np.random.default_rng({"reload": 7300, "reload_verify_first": 7350, "writeback": 7400}[direction])
    sess = si.GcmSession(KEY, SALT, 0, max_record_bytes=70000)
    if direction == "writeback":
        case = _writeback_case
    else:
        case = functools.partial(_reload_case, strict=direction == "reload_verify_first")
    ticket = 1
    try:
        for i in range(14):
            nrec = int(rng.choice([1, 2, 7, 64, 255, 300, 511, 640, 1030]))
            n = int(rng.integers(1, 70000)) if nrec <= 300 else int(rng.integers(1, 9000))
            chunk, straddle = int(rng.choice([1, 2, 3, 5, 8])), int(rng.choice([0, 2, 6, 13]))
            print(f"{direction} case {i}: {nrec} records x {n} B, chunk rows {chunk}, straddle {straddle}",
                  flush=True)
            si.set_chunk_rows(chunk)
            si.set_straddle_rows(straddle)
            case(sess, rng, nrec, n, ticket)
            ticket += nrec
    finally:
        si.set_chunk_rows(si.gcm.DEFAULT_CHUNK_ROWS)
        si.set_straddle_rows(si.gcm.DEFAULT_STRADDLE_ROWS)
