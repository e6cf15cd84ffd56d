"""Host logic of the per-layer drivers, without a GPU: the library is replaced
by a recorder, so these pin what NativeTransfer / D2HTransfer submit and in
which order.

* Causal groups: the reference's own test
  (secure_infer/tests/test_grouped_loading.py) -- 41 blocks in groups of 16
  are submitted tail first as [25, 41), [9, 25), [0, 9), each group inside its
  own layer-group brackets sized 2 * len(group), K before V, every block
  exactly once, the layer index unchanged within the layer
  (native_layerwise.py:96-112).
* Slice streams stripe each group's rows (native_layerwise.py:113-129).
* The mixed codec policy (transport_codec.py:18-19).
"""
import math
from unittest import mock

import pytest
import torch

import secure_infer_amd as si
from secure_infer_amd import gcm


class FakeStream:
    def __init__(self, name):
        self.name = name
        self.cuda_stream = id(self)
        self.waits = []

    def wait_stream(self, other):
        self.waits.append(other.name)


class Recorder:
    """Stands in for libsecure_infer.so: records brackets and swaps."""

    def __init__(self, auth=0):
        self.calls = []
        self.auth = auth

    def secure_infer_recovery_wait_layer_authentication(self, layer):
        self.calls.append(("wait", int(layer)))
        return self.auth

    def secure_infer_h2d_layer_group_begin(self, n):
        self.calls.append(("begin", int(n)))
        return 0

    def secure_infer_h2d_layer_group_end(self):
        self.calls.append(("end",))
        return 0

    def secure_infer_h2d_swap(self, stream, sess, host_base, host_block_bytes, host_nblocks, dev, slot_bytes,
                              nslots, mapping_ptr, n, kind, layer, bits, heads, dim, fail):
        import ctypes as ct
        arr = (ct.c_int64 * (2 * n)).from_address(mapping_ptr.value)
        pairs = [(arr[2 * i], arr[2 * i + 1]) for i in range(n)]
        self.calls.append(("swap", stream.value, kind, layer, bits, pairs, host_nblocks, nslots))
        return 0

    def secure_infer_codec_width(self, bits, heads, dim):
        from secure_infer_amd import _lib
        return _lib.load().secure_infer_codec_width(bits, heads, dim)

    def secure_infer_h2d_prefetch(self, sess, host_base, host_block_bytes, host_nblocks, mapping_ptr, n, kind,
                                  layer, bits, heads, dim):
        import ctypes as ct
        arr = (ct.c_int64 * (2 * n)).from_address(mapping_ptr.value)
        self.calls.append(("prefetch", kind, layer, bits, [(arr[2 * i], arr[2 * i + 1]) for i in range(n)]))
        return 0

    def secure_infer_h2d_prefetch_group(self, sess, k_base, v_base, host_block_bytes, host_nblocks, mapping_ptr, n,
                                        layer, bits, heads, dim):
        # the K swap's prefetch, then the V swap's (the tickets' order)
        self.secure_infer_h2d_prefetch(sess, k_base, host_block_bytes, host_nblocks, mapping_ptr, n, 0, layer,
                                       bits, heads, dim)
        self.calls.append(("prefetch_group_pairs_with_previous",))
        return self.secure_infer_h2d_prefetch(sess, v_base, host_block_bytes, host_nblocks, mapping_ptr, n, 1,
                                              layer, bits, heads, dim)

    def secure_infer_h2d_prefetch_layer(self, sess, k_base, v_base, host_block_bytes, host_nblocks, mapping_ptr,
                                        starts, rows, ngroups, layer, bits, heads, dim):
        import ctypes as ct
        groups = []
        for g in range(ngroups):
            arr = (ct.c_int64 * (2 * rows[g])).from_address(mapping_ptr.value + 16 * starts[g])
            groups.append((starts[g], [(arr[2 * i], arr[2 * i + 1]) for i in range(rows[g])]))
        self.calls.append(("prefetch_layer", layer, bits, groups))
        return 0


def run_transfer(nblocks, group, streams, layer=7, shape=None, nslots=None, keep_prefetch=False,
                 pipeline_seal=True, stripe=False, merge_groups=False, codec_auth_wait=False, auth=0):
    rec = Recorder(auth)
    parent = FakeStream("parent")
    shape = shape or si.LayerShape(2, 64)
    sess = mock.Mock()
    sess._h = None
    nt = si.NativeTransfer(sess, shape, streams=streams or None, causal_group_blocks=group,
                           pipeline_seal=pipeline_seal, stripe=stripe, merge_groups=merge_groups,
                           codec_auth_wait=codec_auth_wait)
    nt.layer = layer
    host = [torch.zeros((nblocks, 4), dtype=torch.int16), torch.zeros((nblocks, 4), dtype=torch.int16)]
    dest = [torch.zeros((nslots or nblocks + 100, 4), dtype=torch.int16) for _ in range(2)]
    mapping = torch.stack((torch.arange(nblocks), torch.arange(nblocks) + 100), dim=1)
    with mock.patch.object(gcm, "lib", return_value=rec), \
         mock.patch.object(gcm, "_dev", lambda t, name: None), \
         mock.patch.object(gcm.torch.cuda, "current_stream", return_value=parent):
        nt.single_layer_kv_transfer((host, mapping), dest, None, False, 2, True, False)
    if not keep_prefetch:
        rec.calls = [c for c in rec.calls if not c[0].startswith("prefetch")]
    return nt, rec, parent


def test_partial_group_preserves_layer_and_mapping():
    nt, rec, _ = run_transfer(41, 16, None)
    begins = [c[1] for c in rec.calls if c[0] == "begin"]
    assert begins == [32, 32, 18]
    assert nt.layer == 8 and nt.causal_group_blocks == 16
    swaps = [c for c in rec.calls if c[0] == "swap"]
    assert all(c[3] == 7 for c in swaps)
    for kind in range(2):
        parts = [c[5] for c in swaps if c[2] == kind]
        assert [len(p) for p in parts] == [16, 16, 9]
        combined = [p for part in parts for p in part]
        assert sorted(h for h, _ in combined) == list(range(41))
        assert all(s == h + 100 for h, s in combined)
    # tail first: the first group holds blocks 25..40
    assert [h for h, _ in swaps[0][5]] == list(range(25, 41))
    # per group: begin, K swap, V swap, end
    kinds = [c[0] if c[0] != "swap" else ("K", "V")[c[2]] for c in rec.calls]
    assert kinds == ["begin", "K", "V", "end"] * 3


def test_record_order_is_layer_group_kind_block():
    """Tickets are handed out in submission order, so the records of a
    48-block layer with LOAD_CHUNK 2048 (16-block groups) take tickets in
    (group from the tail, kind, block) order -- the order
    reference_ticket_order() gives to device-resident wire records."""
    _, rec, _ = run_transfer(48, 16, None, layer=0)
    order = [(c[2], h) for c in rec.calls if c[0] == "swap" for h, _ in c[5]]
    assert order == gcm.reference_ticket_order(48, 16)
    assert order[:3] == [(0, 32), (0, 33), (0, 34)] and order[16] == (1, 32) and order[32] == (0, 16)


def test_slice_streams_stripe_rows_and_join():
    s1, s2 = FakeStream("s1"), FakeStream("s2")
    _, rec, parent = run_transfer(10, 0, [s1, s2], stripe=True)
    swaps = [c for c in rec.calls if c[0] == "swap"]
    assert [(c[1], c[2], len(c[5])) for c in swaps] == [
        (s1.cuda_stream, 0, 5), (s2.cuda_stream, 0, 5), (s1.cuda_stream, 1, 5), (s2.cuda_stream, 1, 5)]
    assert s1.waits == ["parent"] and s2.waits == ["parent"]
    assert parent.waits == ["s1", "s2"]


def test_unstriped_slice_streams_keep_the_striped_ticket_order():
    """Without striping, every row goes to the first slice stream, K then V, in
    the order the stripes would take their tickets; the group is one launch
    and only the stream that carries it is joined."""
    s1, s2 = FakeStream("s1"), FakeStream("s2")
    _, rec_s, _ = run_transfer(10, 0, [s1, s2], stripe=True)
    t1, t2 = FakeStream("s1"), FakeStream("s2")
    _, rec, parent = run_transfer(10, 0, [t1, t2])
    swaps = [c for c in rec.calls if c[0] == "swap"]
    assert [(c[1], c[2], len(c[5])) for c in swaps] == [(t1.cuda_stream, 0, 10), (t1.cuda_stream, 1, 10)]
    order = [(c[2], h) for c in swaps for h, _ in c[5]]
    striped = [(c[2], h) for c in rec_s.calls if c[0] == "swap" for h, _ in c[5]]
    assert order == striped
    assert t1.waits == ["parent"] and t2.waits == [] and parent.waits == ["s1"]


def test_swap_carries_pool_sizes():
    _, rec, _ = run_transfer(5, 0, None, nslots=164)
    swaps = [c for c in rec.calls if c[0] == "swap"]
    assert swaps and all(c[6] == 5 and c[7] == 164 for c in swaps)


@pytest.mark.parametrize("nslots", [64, 104])
def test_out_of_pool_mapping_is_refused_before_sealing_ahead(nslots):
    """Slots 100..104 do not fit a 64- or 104-slot cache: the layer is
    refused before any record is sealed ahead (the swaps would refuse it)."""
    with pytest.raises(RuntimeError):
        run_transfer(5, 0, None, nslots=nslots, keep_prefetch=True)


@pytest.mark.parametrize("layers", [1, 2, 3, 28, 32, 40, 80])
def test_mixed_codec_policy(layers):
    for layer in range(layers):
        want = 8 if layer < math.ceil(layers / 3) else 4
        assert si.layer_bits("mixed", layer, layers) == want
        assert si.layer_bits("int8", layer, layers) == 8
        assert si.layer_bits("int4", layer, layers) == 4
        assert si.layer_bits("none", layer, layers) == 0
    with pytest.raises(ValueError):
        si.layer_bits("fp8", 0, layers)


def test_mixed_shape_bits_reach_the_swap():
    shape = si.LayerShape(2, 64, codec="mixed", layers=3)
    assert [shape.bits_for(l) for l in range(3)] == [8, 4, 4]
    with pytest.raises(ValueError):
        shape.record_bytes
    for layer, bits in ((0, 8), (1, 4), (2, 4)):
        _, rec, _ = run_transfer(4, 0, None, layer=layer, shape=shape)
        assert {c[4] for c in rec.calls if c[0] == "swap"} == {bits}
    with pytest.raises(ValueError):
        si.LayerShape(2, 64, codec="mixed")


def test_layer_seals_are_queued_in_swap_order():
    """pipeline_seal: before its swaps, a layer's records are queued for
    sealing on the host pool part by part in exactly the order (and with the
    exact mappings) the swaps then consume them, so tickets follow the
    reference's (group, kind, block) order either way."""
    _, rec, _ = run_transfer(41, 16, None, layer=3, keep_prefetch=True)
    pre = [(c[1], c[2], c[4]) for c in rec.calls if c[0] == "prefetch"]
    swaps = [(c[2], c[3], c[5]) for c in rec.calls if c[0] == "swap"]
    assert pre == swaps and len(pre) == 6
    # one stream: each group's K and V are sealed as one group prefetch
    assert len([c for c in rec.calls if c[0] == "prefetch_group_pairs_with_previous"]) == 3
    first_swap = next(i for i, c in enumerate(rec.calls) if c[0] == "swap")
    last_prefetch = max(i for i, c in enumerate(rec.calls) if c[0] == "prefetch")
    assert last_prefetch < first_swap


def test_unpipelined_layers_are_sealed_on_demand():
    _, rec, _ = run_transfer(41, 16, None, layer=3, keep_prefetch=True, pipeline_seal=False)
    assert not [c for c in rec.calls if c[0] == "prefetch"]


def test_merged_groups_keep_the_swaps_and_their_order():
    """merge_groups: one layer group of 2 * 41 records around the same swaps,
    in the same order (so the same tickets) as one group per causal group;
    the layer is sealed ahead as one layer prefetch naming every group (tail
    first) before the first swap."""
    _, rec_g, _ = run_transfer(41, 16, None, layer=3)
    _, rec, _ = run_transfer(41, 16, None, layer=3, keep_prefetch=True, merge_groups=True)
    swaps = [c for c in rec.calls if c[0] == "swap"]
    assert [c[2:] for c in swaps] == [c[2:] for c in rec_g.calls if c[0] == "swap"]  # stream handles differ
    kinds = [c[0] if c[0] != "swap" else ("K", "V")[c[2]] for c in rec.calls if not c[0].startswith("prefetch")]
    assert kinds == ["begin"] + ["K", "V"] * 3 + ["end"]
    assert [c[1] for c in rec.calls if c[0] == "begin"] == [82]
    order = [(c[2], h) for c in swaps for h, _ in c[5]]
    assert order == gcm.reference_ticket_order(41, 16)
    pre = [c for c in rec.calls if c[0].startswith("prefetch")]
    assert len(pre) == 1 and pre[0][0] == "prefetch_layer" and pre[0][1:3] == (3, 0)
    groups = pre[0][3]
    assert [(start, len(pairs)) for start, pairs in groups] == [(25, 16), (9, 16), (0, 9)]
    assert [p for _, pairs in groups for p in pairs] == [p for c in swaps if c[2] == 0 for p in c[5]]
    assert rec.calls.index(pre[0]) < next(i for i, c in enumerate(rec.calls) if c[0] == "swap")


def test_merged_single_group_is_a_group_prefetch():
    _, rec, _ = run_transfer(10, 16, None, keep_prefetch=True, merge_groups=True)
    assert [c[0] for c in rec.calls if c[0].startswith("prefetch")] == [
        "prefetch", "prefetch_group_pairs_with_previous", "prefetch"]


@pytest.mark.parametrize("lookahead", [0, 1, 2])
def test_reload_layers_seals_ahead_in_layer_order(lookahead):
    """reload_layers: before layer l's swaps, layers l .. l + lookahead are
    queued for sealing, each once and in layer order (so tickets keep the
    (layer, group, kind, block) order); every layer's swaps then consume
    them, and a mapping outside its pool is refused before anything is
    sealed."""
    rec = Recorder()
    parent = FakeStream("parent")
    shape = si.LayerShape(2, 64)
    sess = mock.Mock()
    sess._h = None
    nt = si.NativeTransfer(sess, shape, causal_group_blocks=16)
    nt.layer = 5
    nb, nlayers = 20, 4
    payloads, dests = [], []
    for _ in range(nlayers):
        host = [torch.zeros((nb, 4), dtype=torch.int16), torch.zeros((nb, 4), dtype=torch.int16)]
        payloads.append((host, torch.stack((torch.arange(nb), torch.arange(nb) + 3), dim=1)))
        dests.append([torch.zeros((nb + 3, 4), dtype=torch.int16) for _ in range(2)])
    with mock.patch.object(gcm, "lib", return_value=rec), \
         mock.patch.object(gcm, "_dev", lambda t, name: None), \
         mock.patch.object(gcm.torch.cuda, "current_stream", return_value=parent):
        nt.reload_layers(payloads, dests, lookahead=lookahead)
        assert nt.layer == 5 + nlayers
        events = []
        for c in rec.calls:
            if c[0] == "prefetch" and c[1] == 0 and (not events or events[-1] != ("P", c[2])):
                events.append(("P", c[2]))
            elif c[0] == "swap" and (not events or events[-1] != ("S", c[3])):
                events.append(("S", c[3]))
        want = []
        queued = set()
        for l in range(nlayers):
            for a in range(l, min(nlayers, l + 1 + lookahead)):
                if a not in queued:
                    queued.add(a)
                    want.append(("P", 5 + a))
            want.append(("S", 5 + l))
        assert events == want
        # the prefetched parts are exactly the swapped ones, layer by layer
        pre = [(c[1], c[2], c[4]) for c in rec.calls if c[0] == "prefetch"]
        sw = [(c[2], c[3], c[5]) for c in rec.calls if c[0] == "swap"]
        assert sorted(pre, key=lambda x: x[1]) == sorted(sw, key=lambda x: x[1]) and len(pre) == len(sw)
        # refused before any sealing
        rec.calls.clear()
        bad = list(payloads)
        bad[2] = (payloads[2][0], torch.stack((torch.arange(nb), torch.arange(nb) + 30), dim=1))
        with pytest.raises(RuntimeError):
            nt.reload_layers(bad, dests, lookahead=lookahead)
        assert not [c for c in rec.calls if c[0] in ("prefetch", "swap")]


@pytest.mark.parametrize("auth", [0, -1], ids=["authenticated", "failed"])
def test_codec_auth_wait(auth):
    """codec_auth_wait: after a codec layer's swaps (all of its groups) the
    transfer waits for that layer's authentication and raises on failure, as
    the reference's codec transfer asserts wait_auth(layer) == 0 before it
    decodes (transport_codec.py:168-174); the layer index has moved on either
    way.  A bf16 layer, or the option off, does not wait."""
    shape = si.LayerShape(2, 64, codec_bits=4)
    if auth == 0:
        nt, rec, _ = run_transfer(41, 16, None, layer=5, shape=shape, codec_auth_wait=True, auth=auth)
        assert rec.calls[-1] == ("wait", 5) and nt.layer == 6
        assert [c[0] for c in rec.calls].count("wait") == 1
        assert [c[0] for c in rec.calls[:-1]].count("swap") == 6  # three groups, K and V
    else:
        with pytest.raises(RuntimeError, match="Packed KV authentication failed"):
            run_transfer(41, 16, None, layer=5, shape=shape, codec_auth_wait=True, auth=auth)
    for sh, on in ((si.LayerShape(2, 64), True), (shape, False)):
        _, rec, _ = run_transfer(41, 16, None, layer=5, shape=sh, codec_auth_wait=on, auth=-1)
        assert not any(c[0] == "wait" for c in rec.calls)
