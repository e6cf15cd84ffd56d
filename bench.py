"""Authenticated KV reload / writeback benchmark on one MI355X.

Workload (default): Llama-3-8B KV shape, 32 layers x 8 kv heads x head_dim 128,
bf16 ~N(0,1), a 6144-token prefix = 48 blocks of 128 tokens, reloaded into a
paged cache of 512 slots per (layer, kind) at a seeded permutation of slots.
One record = one (block, kind) slice of 262,144 B; 96 records per layer.  A
step reloads all 32 layers, one fused verify + decrypt + scatter launch per
layer, with the ciphertext wire records already resident in HBM.  Other
workloads (--config): int8 / int4 codec reloads (the int4 one with 1 % of the
records tampered, which must fail closed), a Llama-3-70B int4 writeback, and
one tensor-parallel rank of Llama-3-70B at TP = 8 (1 kv head x 128, 32-KiB
records) reloaded (bf16) and written back (int4).

Prints ONE JSON line.  `value` is GB/s of algorithmic bytes over the timed
region (reload, per record: ciphertext read + bf16 write + tag + AAD + status;
writeback: bf16 read + ciphertext write + tag + AAD).  `roofline.achieved` is
the same bytes over `roofline.kernel_us`, the median kernel time of one
layer's launch sequence measured in this run (one more back-to-back pass
after the timed region whose kernels stamp the device clock at the start and
end of every wave).  `roofline.traffic` and `issue`
(VALU / LDS issue fractions of the GCM kernel) come from the committed
rocprofv3 counter summaries under profiles/.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "authenticated KV reload GB/s and μs/layer (1 GPU); % of HBM peak"

CONFIGS = {
    # name: direction, layers, kv_heads, head_dim, blocks, slots, codec bits, tampered fraction
    "reload_bf16_llama3_8b_6144tok": dict(op="reload", layers=32, heads=8, dim=128, blocks=48, slots=512,
                                          bits=0, tamper=0.0),
    "reload_int8_llama3_8b_8192tok": dict(op="reload", layers=32, heads=8, dim=128, blocks=64, slots=512,
                                          bits=8, tamper=0.0),
    "reload_int4_qwen2_5_7b_8192tok": dict(op="reload", layers=28, heads=4, dim=128, blocks=64, slots=512,
                                           bits=4, tamper=0.01),
    "writeback_int4_llama3_70b_32768tok": dict(op="writeback", layers=80, heads=8, dim=128, blocks=256,
                                               slots=512, bits=4, tamper=0.0),
    # One rank of Llama-3-70B at tensor parallelism 8: 1 kv head x 128 per
    # rank, so 32-KiB bf16 records (10,256-B int4 packets), 512 per layer.
    "reload_bf16_llama3_70b_tp8_rank_32768tok": dict(op="reload", layers=80, heads=1, dim=128, blocks=256,
                                                     slots=512, bits=0, tamper=0.0),
    "writeback_int4_llama3_70b_tp8_rank_32768tok": dict(op="writeback", layers=80, heads=1, dim=128,
                                                        blocks=256, slots=512, bits=4, tamper=0.0),
}
DEFAULT = "reload_bf16_llama3_8b_6144tok"
# RUNTIME_LOAD_CHUNK of the reference's reuse connectors (connector.py:21, 288):
# a layer's reload is submitted in groups of 2048 / 128 = 16 blocks, tail first.
LOAD_CHUNK_BLOCKS = 2048 // 128


class Range:
    """A named ROCTx range (rocprofiler-sdk's roctx library) around one part
    of the run -- a workload, its timed region, its per-launch kernel pass --
    so that a kernel trace of this same command taken with --marker-trace
    splits per workload and phase.  Costs a library call per range; does
    nothing where the library is absent."""
    _fns = None

    def __init__(self, name: str):
        self.name = name.encode()

    @classmethod
    def _load(cls):
        if cls._fns is None:
            import ctypes as ct
            try:
                lib = ct.CDLL("librocprofiler-sdk-roctx.so.1")
                lib.roctxRangePushA.argtypes, lib.roctxRangePushA.restype = [ct.c_char_p], ct.c_int
                lib.roctxRangePop.argtypes, lib.roctxRangePop.restype = [], ct.c_int
                cls._fns = (lib.roctxRangePushA, lib.roctxRangePop)
            except (OSError, AttributeError):
                cls._fns = ()
        return cls._fns

    def __enter__(self):
        fns = self._load()
        if fns:
            fns[0](self.name)
        return self

    def __exit__(self, *exc):
        fns = self._load()
        if fns:
            fns[1]()
        return False


def aad_bytes(direction: int, kind: int, layer: int, block_id: int, nbytes: int, ticket: int) -> bytes:
    """Reference AAD layout (secure_infer_build_gcm_aad, secure_infer.cpp:730-775)."""
    out = bytearray(64)
    out[0:8] = b"SFAD" + bytes([1, direction, kind & 0xFF, 0])
    out[8:12] = layer.to_bytes(4, "big")
    out[12:20] = block_id.to_bytes(8, "big")
    out[28:36] = nbytes.to_bytes(8, "big")
    out[36:44] = ticket.to_bytes(8, "big")
    return bytes(out)


def record_tickets(op: str, nblocks: int, ticket0: int) -> np.ndarray:
    """Ticket of each record of a layer (records K blocks then V blocks).
    Reload follows NativeTransfer's submission order (groups of
    LOAD_CHUNK_BLOCKS from the tail, K then V, native_layerwise.py:96-129);
    writeback follows the D2H branch's (all K blocks, then all V blocks,
    npu_predict.py:895-906)."""
    from secure_infer_amd.gcm import reference_ticket_order
    if op == "writeback":
        return ticket0 + np.arange(2 * nblocks, dtype=np.int64)
    pos = {kb: i for i, kb in enumerate(reference_ticket_order(nblocks, LOAD_CHUNK_BLOCKS))}
    return ticket0 + np.array([pos[divmod(r, nblocks)] for r in range(2 * nblocks)], np.int64)


def iv_words_of(salt: bytes, nonce: int, tickets: np.ndarray) -> np.ndarray:
    """salt || BE64(nonce + ticket) || BE32(2) as four big-endian words
    (secure_infer_derive_transfer_iv, secure_infer.cpp:274-300)."""
    t = (np.uint64(nonce) + tickets.astype(np.uint64))
    w = np.zeros((tickets.size, 4), np.uint32)
    w[:, 0] = int.from_bytes(salt[:4], "big")
    w[:, 1] = (t >> np.uint64(32)).astype(np.uint32)
    w[:, 2] = (t & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    w[:, 3] = 2
    return w


def cpu_check_sampled_layers(op, layers, blocks_host, cache, wire, slots, tampered, key, salt, tickets, H, D, NB,
                         bits, nbytes, stride, tag_off, torch):
    """Bit-exactness of the timed work on sampled layers against the oracle:
    reload -> the cache holds decode(encode(original)) (bf16: the original),
    zeros for tampered records; writeback -> every record's ciphertext and tag
    equal OpenSSL's over the oracle's packet."""
    from oracle import oracle as O
    ok = True
    for layer in layers:
        orig = blocks_host[layer]  # [2, NB, 128, H, D] uint16
        if op == "reload":
            want = orig.copy()
            if bits:
                for k in range(2):
                    for b in range(NB):
                        want[k, b] = O.codec_decode(O.codec_encode(orig[k, b], bits, k, layer), H, D, bits, k)
            for l2, r in tampered:
                if l2 == layer:
                    want[r // NB, r % NB] = 0
            got = torch.stack([cache[layer, k][slots[layer]] for k in range(2)])
            ok &= bool(torch.equal(got.view(torch.int16),
                                   torch.from_numpy(want.view(np.int16)).to(got.device)))
        else:
            ww = wire[layer].cpu().numpy().reshape(2 * NB, stride)
            for r in range(2 * NB):
                k, b = divmod(r, NB)
                t = int(tickets[layer][r])
                pkt = O.codec_encode(orig[k, b], bits, k, layer) if bits else orig[k, b].view(np.uint8).reshape(-1)
                aad = O.build_gcm_aad(2, k, layer, b, 0, nbytes, t)
                iv12 = salt[:4] + t.to_bytes(8, "big")
                c, tag = O.ossl_gcm_encrypt(key, iv12, aad, pkt)
                ok &= bool(np.array_equal(ww[r, :nbytes], c) and ww[r, tag_off:tag_off + 16].tobytes() == tag)
    return ok


def algorithmic_bytes_per_record(op: str, record_bytes: int, block_bytes: int) -> int:
    if op == "reload":  # ciphertext read + bf16 write + tag 16 + AAD 64 + status 4
        return record_bytes + block_bytes + 16 + 64 + 4
    return block_bytes + record_bytes + 16 + 64  # bf16 read + ciphertext write + tag + AAD


def load_traffic(workload: str):
    path = ROOT / "profiles" / f"{workload}_traffic.json"
    if path.exists():
        try:
            d = json.loads(path.read_text())
            return d.get("traffic_bytes_per_launch")
        except Exception:
            return None
    return None


def load_issue(workload: str):
    """VALU / LDS issue fractions of the workload's GCM kernel from the committed
    rocprofv3 counter summary (profiles/<workload>_issue.json), or None."""
    path = ROOT / "profiles" / f"{workload}_issue.json"
    if not path.exists():
        return None
    try:
        d = json.loads(path.read_text())
    except Exception:
        return None
    for kernel, row in d.items():
        if "gcm_records_kernel" in kernel:
            return {"kernel": kernel, "valu_issue_frac": row.get("valu_issue_frac"),
                    "lds_active_frac": row.get("lds_active_frac"),
                    "lds_bank_conflict_frac": row.get("lds_bank_conflict_frac"),
                    "valu_busy_rocprof_pct": row.get("valu_busy_rocprof_pct"),
                    "source": f"profiles/{workload}_issue.md"}
    return None


def cpu_baseline(op: str, wire_host: np.ndarray, stride: int, nbytes: int, nrec: int, n_k: int,
                 key: bytes, ivs: np.ndarray, heads: int, dim: int, bits: int, layer: int,
                 budget_s: float, algo_per_layer: int, planes, gpu_wire: np.ndarray | None):
    """OpenSSL EVP AES-128-GCM on the host cores over the same records as the
    GPU: reload = decrypt + verify + (decode) + scatter into a host paged cache;
    writeback = gather + (encode) + encrypt + tag from one."""
    from oracle import oracle as O
    lib = O.ossl()
    threads = len(os.sched_getaffinity(0))
    slot_bytes = 128 * heads * dim * 2
    nb = max(n_k, 1)
    slots = np.arange(nrec, dtype=np.int64) % nb
    kinds = np.array([0] * n_k + [1] * (nrec - n_k), np.uint32)
    if op == "reload":
        cache = [np.zeros(nb * slot_bytes, np.uint8) for _ in range(2)]
    else:
        cache = [np.ascontiguousarray(planes[k]).reshape(-1).copy() for k in range(2)]
    status = np.zeros(nrec, np.uint32)
    iv12 = np.ascontiguousarray(
        np.stack([ivs[:, w].astype(">u4").view(np.uint8).reshape(-1, 4) for w in range(3)], 1)
        .reshape(nrec, 12))
    tag_off = (nbytes + 31) & ~31
    direction = 1 if op == "reload" else 2

    def run(nthr):
        return lib.si_ossl_layer(direction, O._ptr(np.frombuffer(key, np.uint8).copy()), O._ptr(iv12),
                                 O._ptr(wire_host), stride, nbytes, tag_off, tag_off + 32, nrec,
                                 O._ptr(cache[0]), O._ptr(cache[1]), slot_bytes, O._ptr(slots),
                                 O._ptr(kinds), bits, heads, dim, layer, O._ptr(status), nthr)

    run(threads)  # warm-up (and the result that is compared with the GPU's)
    if op == "reload":
        gst = gpu_wire.reshape(nrec, stride)[:, tag_off + 16:tag_off + 20].copy().view("<u4").ravel()
        ok = bool(np.array_equal(status, gst))  # same accept / reject decision per record
        same = all(np.array_equal(cache[k].reshape(-1, slot_bytes)[i], planes[k][i])
                   for k in range(2) for i in range(n_k))
    else:
        ok = True
        w = wire_host.reshape(nrec, stride)
        g = gpu_wire.reshape(nrec, stride)
        same = bool(np.array_equal(w[:, :nbytes], g[:, :nbytes]) and
                    np.array_equal(w[:, tag_off:tag_off + 16], g[:, tag_off:tag_off + 16]))
    times = []
    t_end = time.time() + budget_s
    while time.time() < t_end or len(times) < 5:
        times.append(run(threads) / 1e9)
        if len(times) >= 20000:
            break
    t1 = [run(1) / 1e9 for _ in range(3)]
    med = float(np.median(times))
    what = ("decrypt+verify" + ("+decode" if bits else "") + "+scatter") if op == "reload" else \
           ("gather" + ("+encode" if bits else "") + "+encrypt+tag")
    return dict(value=round(algo_per_layer / med / 1e9, 3), unit="GB/s", cores=threads,
                kind="port",
                sample=(f"OpenSSL {lib.si_ossl_version().decode()} EVP_aes_128_gcm {what} of one layer "
                        f"({nrec} records x {nbytes} B) x {len(times)} reps, median; 1 thread: "
                        f"{round(algo_per_layer / float(np.median(t1)) / 1e9, 3)} GB/s"),
                us_per_layer=round(med * 1e6, 1), statuses_match_gpu=ok, matches_gpu=bool(same))


def ledger_split(path: Path, steps: int) -> dict:
    """Mean host seal / H2D copy / kernel microseconds per layer from the
    library's H2D ledger rows (SECURE_INFER_H2D_PROFILE, one row per launch:
    a causal group's K and V swaps go out as one), by record source."""
    if not path.exists():
        return {}
    rows = [l.split(",") for l in path.read_text().strip().splitlines()[1:]]
    out = {}
    for src in ("sealed", "prefetched", "prefetch_waited"):
        sel = [r for r in rows if r[4] == src]
        if not sel:
            continue
        per_layer = len(sel) / max(len({r[0] for r in sel}) * steps, 1)  # causal groups
        out[src] = {"launches": len(sel), "launches_per_layer": round(per_layer, 2)}
        for col, name in ((5, "seal_us"), (6, "h2d_copy_us"), (7, "kernel_us")):
            out[src][name + "_per_layer"] = round(float(np.mean([float(r[col]) for r in sel])) * per_layer, 1)
    return out


def end_to_end(si, torch, sess, op, cfg, cache, slots, nbytes, block_bytes, algo_layer, steps, truth,
               slice_streams=1, stripe=False):
    """The same layers through the host-memory path: reload = host OpenSSL seal
    into the pinned ring, H2D on the library's copy stream, fused kernel;
    writeback = fused kernel, D2H, host authentication into host pools.  Wall
    time of whole steps after one warm-up step (PCIe included; never `value`).
    Reload is timed twice: records sealed on demand by each swap, and every
    layer's records sealed ahead of demand (secure_infer_h2d_prefetch) before
    the step -- the reload latency once the host has pre-sealed a stored
    prefix.  The library's ledger splits both into host seal, H2D copy and
    kernel time per layer."""
    L, H, D, NB, bits = cfg["layers"], cfg["heads"], cfg["dim"], cfg["blocks"], cfg["bits"]
    shape = si.LayerShape(H, D, bits)
    dev = cache.device
    mapping_rl = [torch.stack([torch.arange(NB), slots[l].cpu()], 1).contiguous() for l in range(L)]
    if bits == 0:
        pool = lambda: torch.zeros((NB, 128, H, D), dtype=torch.bfloat16)
    else:
        pool = lambda: torch.zeros((NB, nbytes), dtype=torch.uint8)
    hosts = [(pool(), pool()) for _ in range(L)]
    si.clear_host_ranges()
    for l in range(L):
        si.register_host_range(hosts[l][0], l, 0)
        si.register_host_range(hosts[l][1], l, 1)
    d2h = si.D2HTransfer(sess, shape, group_blocks=16)  # PIPE_D2H_GROUP_BLOCKS default (npu_predict.py:88-94)
    wb_map = [torch.stack([slots[l].cpu(), torch.arange(NB)], 1).contiguous() for l in range(L)]
    # host pools hold what a writeback produced (bf16 blocks or codec packets)
    for l in range(L):
        d2h.store([(cache[l, 0], cache[l, 1])], [hosts[l]], wb_map[l], layers=[l])
    out = {"host_threads": int(si._lib.load().secure_infer_host_threads())}
    if op == "reload":
        cache.zero_()
        # Slice streams as the reference's PIPE_GCM_H2D_SLICE_STREAMS (npu_predict.py:130-155):
        # 1 = the caller's stream only; more, with `stripe`, stripe each
        # group's swaps over side streams that the caller's stream joins.
        streams = [torch.cuda.Stream() for _ in range(slice_streams)] if slice_streams > 1 else None
        nt = si.NativeTransfer(sess, shape, streams=streams, causal_group_blocks=LOAD_CHUNK_BLOCKS,
                               stripe=stripe)
        out["slice_streams"] = slice_streams
        out["stripe"] = bool(stripe)
        lib = si._lib.load()

        layers_in = [(hosts[l], mapping_rl[l]) for l in range(L)]
        layers_out = [(cache[l, 0], cache[l, 1]) for l in range(L)]

        def step(mode):
            """One reload of every layer: "on_demand" (each layer sealed as its
            transfer comes), "sealed_ahead" (every layer sealed before the
            step), "layer_ahead" (reload_layers: layer l + 1 seals while
            layer l copies)."""
            nt.layer = 0
            if mode == "sealed_ahead":
                queued = [nt.prefetch_kv_transfer(layers_in[l], l) for l in range(L)]
                if not all(queued):
                    raise RuntimeError("prefetch budget (SECURE_INFER_PREFETCH_MB) too small for every layer")
                deadline = time.perf_counter() + 120
                while int(lib.secure_infer_count_ready_unconsumed_gcm_tickets()) < L * 2 * NB:
                    if time.perf_counter() > deadline:
                        raise RuntimeError("prefetched records not sealed within 120 s")
                    time.sleep(0.0005)
            t0 = time.perf_counter()
            if mode == "layer_ahead":
                nt.reload_layers(layers_in, layers_out, lookahead=1)
            else:
                for l in range(L):
                    nt.single_layer_kv_transfer(layers_in[l], layers_out[l])
            issue[mode] = issue.get(mode, []) + [time.perf_counter() - t0]
            good = all(nt.wait_layer(l) == 0 for l in range(L))
            torch.cuda.synchronize()
            return good, time.perf_counter() - t0

        issue = {}  # host time to issue every layer (the transfer calls' return), per mode

        def timed(mode, merge):
            """Median step of `steps` and the prefetch counters they moved
            (busy_fallback: swaps that waited for their records' sealing)."""
            nonlocal ok
            nt.merge_groups = merge
            s0 = si.transfer_prefetch_stats()
            issue.pop(mode, None)
            times = []
            with Range(f"e2e:{mode}{':merged' if merge else ''}"):
                for _ in range(steps):
                    good, t = step(mode)
                    ok &= good
                    times.append(t)
            s1 = si.transfer_prefetch_stats()
            nt.merge_groups = False
            issued[mode + (":merged" if merge else "")] = round(float(np.median(issue[mode])) * 1e6 / L, 1)
            return float(np.median(times)), {k: s1[k] - s0[k] for k in s1}

        issued = {}  # median host issue time per layer, per mode

        def matches_truth():
            if truth is None:
                return True
            got = torch.stack([cache[l][:, slots[l]] for l in range(L)])
            return bool(torch.equal(got.view(torch.int16), truth.view(torch.int16)))

        # Timed steps run with the ledger paused (its timing events cost the
        # host ~10 us per launch); one more step of each mode records it.
        si.pause_h2d_profile(True)
        ok, _ = step("on_demand")
        med, stats = {}, {}
        for mode in ("on_demand", "sealed_ahead", "layer_ahead"):
            med[mode], stats[mode] = timed(mode, False)
        dt = med["on_demand"]
        ok &= matches_truth()
        out["on_demand_prefetch_stats"] = stats["on_demand"]
        out["sealed_ahead_of_demand"] = {"us_per_layer": round(med["sealed_ahead"] * 1e6 / L, 1),
                                         "GB_s": round(algo_layer * L / med["sealed_ahead"] / 1e9, 2),
                                         "prefetch_stats": stats["sealed_ahead"]}
        out["sealed_one_layer_ahead"] = {"us_per_layer": round(med["layer_ahead"] * 1e6 / L, 1),
                                         "GB_s": round(algo_layer * L / med["layer_ahead"] / 1e9, 2),
                                         "prefetch_stats": stats["layer_ahead"]}
        # The same steps with each layer's causal groups merged into one
        # launch (NativeTransfer merge_groups: same swaps, same tickets; one
        # layer prefetch and one DMA when sealed ahead).
        cache.zero_()
        merged = {}
        for mode in ("on_demand", "sealed_ahead", "layer_ahead"):
            merged[mode], stats["merged_" + mode] = timed(mode, True)
        ok &= matches_truth()
        out["merged_layer_launch"] = {
            "on_demand_us_per_layer": round(merged["on_demand"] * 1e6 / L, 1),
            "sealed_ahead_us_per_layer": round(merged["sealed_ahead"] * 1e6 / L, 1),
            "sealed_ahead_GB_s": round(algo_layer * L / merged["sealed_ahead"] / 1e9, 2),
            "one_layer_ahead_us_per_layer": round(merged["layer_ahead"] * 1e6 / L, 1),
            "one_layer_ahead_GB_s": round(algo_layer * L / merged["layer_ahead"] / 1e9, 2),
            "one_layer_ahead_prefetch_stats": stats["merged_layer_ahead"]}
        # Host time to issue a layer (the transfer calls until they return; the
        # copies and kernels they queue run on): a mode whose figure nears its
        # step time per layer is bound by the host's issue rate.
        out["host_issue_us_per_layer"] = issued
        ledger = os.environ.get("SECURE_INFER_H2D_PROFILE")
        if ledger:
            si.pause_h2d_profile(False)
            split = {}
            for mode, merge, name in (("on_demand", False, "on_demand"),
                                      ("sealed_ahead", False, "sealed_ahead_of_demand"),
                                      ("sealed_ahead", True, "merged_sealed_ahead_of_demand"),
                                      ("layer_ahead", True, "merged_one_layer_ahead")):
                si.drain_h2d_profile_after_job()
                if Path(ledger).exists():
                    Path(ledger).write_text(Path(ledger).read_text().splitlines()[0] + "\n")
                nt.merge_groups = merge
                good, t = step(mode)
                nt.merge_groups = False
                ok &= good
                si.drain_h2d_profile_after_job()
                split[name] = ledger_split(Path(ledger), 1)
                split[name]["step_us_per_layer_with_ledger"] = round(t * 1e6 / L, 1)
            out["ledger_split"] = split
        what = ("host OpenSSL seal + pinned ring + H2D (copy stream) + fused verify/decrypt/scatter, "
                "causal groups of %d blocks; median step" % LOAD_CHUNK_BLOCKS)
    else:
        # One batch per step over every layer with one block table, as the
        # reference's store job submits them (npu_predict.py:874-916).
        ok = True
        srcs = [(cache[l, 0], cache[l, 1]) for l in range(L)]
        d2h.store(srcs, hosts, wb_map[0], layers=list(range(L)))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            d2h.store(srcs, hosts, wb_map[0], layers=list(range(L)))
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        what = ("fused gather/quantise/seal + D2H + host OpenSSL authenticate/decrypt into host pools, "
                "one batch of every layer in groups of %d blocks" % d2h.group_blocks)
    si.clear_host_ranges()
    out.update({"us_per_layer": round(dt * 1e6 / L, 1), "GB_s": round(algo_layer * L / dt / 1e9, 2),
                "steps": steps, "ok": bool(ok), "path": what})
    return out


def run_workload(name: str, args, torch, si, steps: int, warmup: int, with_cpu: bool, cpu_budget: float,
                 e2e_steps: int) -> dict:
    """One workload: set-up (wire records made on the device), `warmup`
    untimed steps, `steps` timed steps of one launch sequence per layer, the
    per-launch kernel pass, correctness, and optionally the CPU leg (oracle
    check of sampled layers + OpenSSL baseline) and the end-to-end leg."""
    cfg = CONFIGS[name]
    op = cfg["op"]
    L, H, D, NB, NS, bits = cfg["layers"], cfg["heads"], cfg["dim"], cfg["blocks"], cfg["slots"], cfg["bits"]
    if args.chunk_rows:
        si.set_chunk_rows(args.chunk_rows)
    if args.straddle_rows >= 0:
        si.set_straddle_rows(args.straddle_rows)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(1234)
    rng = np.random.default_rng(1234)
    key = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
    salt = rng.integers(0, 256, 4, dtype=np.uint8).tobytes()
    block_bytes = 128 * H * D * 2
    nbytes = block_bytes if bits == 0 else si.codec_width(bits, H, D)
    nrec, n_k = 2 * NB, NB
    stride = si.wire_stride(nbytes)
    tag_off = si.wire_tag_offset(nbytes)
    sess = si.GcmSession(key, salt, 0, max_record_bytes=nbytes)
    direction = 1 if op == "reload" else 2

    # paged caches [L, 2, NS, 128, H, D] bf16 and per-layer slot tables (seeded
    # permutations of the slots; K records then V records)
    cache = torch.zeros((L, 2, NS, 128, H, D), dtype=torch.bfloat16, device=dev)
    slots = torch.stack([torch.randperm(NS, generator=gen, device=dev)[:NB] for _ in range(L)])
    slots2 = torch.cat([slots, slots], 1).contiguous()
    for layer in range(L):
        cache[layer, :, slots[layer]] = torch.randn((2, NB, 128, H, D), generator=gen, device=dev,
                                                    dtype=torch.float32).to(torch.bfloat16)

    # Wire records with host-built AADs.  Reload: the ciphertext is made by
    # the GPU writeback path (bit-exact with OpenSSL, checked by the tests)
    # under the tickets a reload of this layer takes in the reference's order.
    wire = torch.zeros((L, nrec * stride), dtype=torch.uint8, device=dev)
    ticket0 = 1
    tickets = [record_tickets(op, NB, ticket0 + layer * nrec) for layer in range(L)]
    ivw = torch.from_numpy(np.stack([iv_words_of(salt, 0, t) for t in tickets])).to(dev)
    aads = np.zeros((L, nrec, 64), np.uint8)
    for layer in range(L):
        for r in range(nrec):
            t = int(tickets[layer][r])
            aads[layer, r] = np.frombuffer(aad_bytes(direction, 0 if r < n_k else 1, layer, r % NB, nbytes, t),
                                           np.uint8)
    wv = wire.view(L, nrec, stride)
    wv[:, :, tag_off + 32:tag_off + 96] = torch.from_numpy(aads).to(dev)
    staging = torch.zeros(nrec * tag_off, dtype=torch.uint8, device=dev) if bits else None
    fails = torch.zeros(L, dtype=torch.int32, device=dev)

    # Each layer's launch is prepared once (descriptor built and checked), as
    # a serving loop with fixed buffers does; a step only calls the library.
    launch_stream = si.gcm._stream(None)
    wb_prep = [sess.prepare_writeback_layer(wire[layer], nbytes, nrec, n_k, cache[layer, 0], cache[layer, 1],
                                            slots2[layer], iv_words_dev=ivw[layer], codec_bits=bits, heads=H,
                                            head_dim=D, layer=layer, staging=staging) for layer in range(L)]
    rl_prep = [sess.prepare_reload_layer(wire[layer], nbytes, nrec, n_k, cache[layer, 0], cache[layer, 1],
                                         slots2[layer], iv_words_dev=ivw[layer], codec_bits=bits, heads=H,
                                         head_dim=D, layer=layer, staging=staging,
                                         fail_count=fails[layer:layer + 1],
                                         verify_before_release=args.verify_before_release) for layer in range(L)]

    def writeback_layer(layer):
        wb_prep[layer].launch(launch_stream)

    def reload_layer(layer):
        rl_prep[layer].launch(launch_stream)

    sample_layers = sorted({0, L // 2, L - 1})
    blocks_host = {l: torch.stack([cache[l, k][slots[l]] for k in range(2)]).view(torch.int16).cpu().numpy()
                   .view(np.uint16) for l in sample_layers}

    tampered = []
    if op == "reload":
        for layer in range(L):
            writeback_layer(layer)
        torch.cuda.synchronize()
        if cfg["tamper"]:
            # seeded records with one seeded ciphertext byte flipped: they must fail closed
            ntam = max(1, round(cfg["tamper"] * L * nrec))
            picks = rng.choice(L * nrec, ntam, replace=False)
            for p in picks:
                layer, r = divmod(int(p), nrec)
                off = int(rng.integers(0, nbytes))
                wv[layer, r, off] ^= 0x5A
                tampered.append((layer, r))
        if bits == 0:
            truth = torch.stack([cache[l][:, slots[l]] for l in range(L)]).clone()
        cache.zero_()
        step = reload_layer
    else:
        step = writeback_layer
    torch.cuda.synchronize()

    for _ in range(warmup):
        for layer in range(L):
            step(layer)
    torch.cuda.synchronize()
    fails.zero_()
    # Clock stamps of the kernel pass that follows the timed region (made
    # now, so that the pass starts as soon as the region ends).
    import ctypes as ct
    lib = si._lib.load()
    words = 1 << 17  # per layer: two words per wave of its kernels
    stamps = torch.empty((L, words), dtype=torch.int64, device=dev)
    stamps[:, 0::2] = torch.iinfo(torch.int64).max
    stamps[:, 1::2] = 0
    khz = ct.c_uint64()
    if lib.secure_infer_gpu_clock_rate_khz(ct.byref(khz)) != 0:
        raise RuntimeError("secure_infer_gpu_clock_rate_khz failed")

    # Timed region: K steps of one launch per layer on one stream, nothing
    # else queued; the average launch duration is the region over K*L.
    stream = torch.cuda.current_stream()
    t_start, t_stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with Range(f"timed:{name}"):
        t_start.record(stream)
        for _ in range(steps):
            for layer in range(L):
                step(layer)
        t_stop.record(stream)
        torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_stop)
    ms_per_step = total_ms / steps
    us_launch = total_ms * 1e3 / (steps * L)

    # The kernel time per launch, measured in this run: one more pass of the
    # same prepared launches right after the timed region (at the clocks the
    # region's sustained load has reached; the correctness checks come after
    # it, on the failure counts the region left), back to back as in the
    # region (same results: reloads rewrite the same plaintext, writebacks the
    # same ciphertext).  Every wave of each layer's kernels writes the
    # device's constant-rate clock when it starts and when it ends
    # (secure_infer_gpu_clock_next_layers, armed once for all layers so the
    # host issues exactly the timed region's calls); a layer's kernel time is
    # its last wave end minus its first wave start.  (HIP events recorded by
    # the launch itself, hipExtLaunchKernel, lengthened each launch they timed
    # by 3-4 us in a kernel trace; arming layer by layer left host gaps of
    # ~9 us, after which a kernel ran ~3 us longer.)  roofline.frac derives
    # from the median; `value` and us_per_layer stay the timed region's
    # figures.
    fails_timed = fails.clone()
    torch.cuda.synchronize()
    if lib.secure_infer_gpu_clock_next_layers(ct.c_void_p(stamps.data_ptr()), words, L) != 0:
        raise RuntimeError("secure_infer_gpu_clock_next_layers failed")
    with Range(f"kernel_pass:{name}"):
        for layer in range(L):
            step(layer)
        torch.cuda.synchronize()
    used_c = (ct.c_uint64 * L)()
    if lib.secure_infer_gpu_clock_layers_used(used_c, L) != 0:
        raise RuntimeError("a kernel's clock stamps did not fit")
    used = list(used_c)
    if len(set(used)) != 1 or used[0] == 0:
        raise RuntimeError(f"clocked layers took different stamp counts: {sorted(set(used))}")
    starts, ends = stamps[:, 0:used[0]:2], stamps[:, 1:used[0]:2]
    if bool((starts == torch.iinfo(torch.int64).max).any()) or bool((ends == 0).any()):
        raise RuntimeError("a wave of a clocked layer wrote no stamp")

    # correctness of what was timed: every layer on the device (bf16 reload),
    # sampled layers against the oracle (every workload)
    nfail = int(fails_timed.sum().item()) if op == "reload" else 0
    exact = True
    if op == "reload" and bits == 0:
        got = torch.stack([cache[l][:, slots[l]] for l in range(L)])
        if tampered:
            for layer, r in tampered:
                k, b = divmod(r, NB)
                truth[layer, k, b] = 0
        exact = bool(torch.equal(got.view(torch.int16), truth.view(torch.int16)))

    tamper_ok = None
    if op == "reload" and tampered:
        zeroed = all(bool((cache[l, r // NB, slots[l, r % NB]] == 0).all()) for l, r in tampered)
        tamper_ok = nfail == len(tampered) * steps and zeroed

    ticks = (ends.max(1).values - starts.min(1).values).cpu().numpy()
    per_launch_us = ticks.astype(np.float64) * 1e3 / khz.value
    kernel_us = float(np.median(per_launch_us))

    algo_layer = nrec * algorithmic_bytes_per_record(op, nbytes, block_bytes)
    gbs = algo_layer * L / (ms_per_step * 1e-3) / 1e9
    achieved = algo_layer / (kernel_us * 1e-6) / 1e9
    res = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded torch.randn bf16 KV, seeded key/salt; ciphertext produced on device)",
        "config": {"workload": name, "direction": op, "layers": L, "kv_heads": H, "head_dim": D,
                   "tokens": NB * 128, "blocks": NB, "records_per_layer": nrec,
                   "record_bytes": nbytes, "cache_slots": NS, "codec_bits": bits,
                   "tampered_records": len(tampered), "algorithmic_bytes_per_layer": algo_layer,
                   **({"verify_before_release": True} if args.verify_before_release else {})},
        "us_per_layer": round(us_launch, 3),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "failed_records_per_step": nfail // max(steps, 1),
        "bit_exact": exact,
        "bit_exact_checked": ("every layer on the device + " if (op == "reload" and bits == 0) else "") +
                             f"layers {sample_layers} against the oracle in the CPU leg" +
                             (" (decode(encode(original)))" if bits and op == "reload" else "") +
                             (" (OpenSSL over the oracle's packets)" if op == "writeback" else ""),
        "ticket_order": ("reload groups of %d blocks from the tail, K then V (reference NativeTransfer)"
                         % LOAD_CHUNK_BLOCKS) if op == "reload" else "K blocks then V blocks (reference D2H)",
        "tamper_fail_closed": tamper_ok,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(name),
                     "kernel_us": round(kernel_us, 3),
                     "kernel_us_range": [round(float(per_launch_us.min()), 3), round(float(per_launch_us.max()), 3)],
                     "kernel_us_source": (f"median over {L} layers of one back-to-back pass after the timed region: "
                                          "per layer, the device clock (wall_clock64, "
                                          f"{khz.value // 1000} MHz) at the end of its kernels' last wave minus "
                                          "the start of their first"),
                     "region_us_per_launch": round(us_launch, 3)},
        "issue": load_issue(name),
    }
    if with_cpu:
        # The CPU leg: the oracle checks the timed work on sampled layers, then
        # OpenSSL on the host cores is timed on one layer.
        res["bit_exact"] = exact and cpu_check_sampled_layers(
            op, sample_layers, blocks_host, cache, wire, slots, tampered, key, salt, tickets, H, D, NB, bits, nbytes,
            stride, tag_off, torch)
        layer = 0
        ivs = ivw[layer].cpu().numpy()
        planes = [cache[layer, k][slots[layer]].view(torch.uint8).reshape(NB, -1).cpu().numpy()
                  for k in range(2)]
        gw = wire[layer].cpu().numpy()
        wh = gw.copy()
        if op == "writeback":
            wh.reshape(nrec, stride)[:, :tag_off + 16] = 0  # the host recomputes ciphertext and tags
        res["cpu_baseline"] = cpu_baseline(op, wh, stride, nbytes, nrec, n_k, key, ivs, H, D, bits, layer,
                                           cpu_budget, algo_layer, planes, gw)
    if e2e_steps > 0:
        if op == "reload" and "SECURE_INFER_H2D_PROFILE" not in os.environ:
            # read by the library at the first H2D swap, which comes later
            import tempfile
            os.environ["SECURE_INFER_H2D_PROFILE"] = os.path.join(tempfile.mkdtemp(), "h2d_ledger.csv")
        with Range(f"end_to_end:{name}"):
            res["end_to_end"] = end_to_end(si, torch, sess, op, cfg, cache, slots, nbytes, block_bytes, algo_layer,
                                           e2e_steps, truth if (op == "reload" and bits == 0) else None,
                                           max(1, min(args.slice_streams, 8)), args.stripe)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default=DEFAULT, choices=sorted(CONFIGS))
    ap.add_argument("--chunk-rows", type=int, default=0)
    ap.add_argument("--straddle-rows", type=int, default=-1,
                    help="straddle cost of the record kernel's share layout (default: the library's)")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--e2e-steps", type=int, default=3,
                    help="steps of the host-memory path (host seal + pinned ring + PCIe); 0 = skip")
    ap.add_argument("--slice-streams", type=int, default=1,
                    help="slice streams of the end-to-end reload (the reference's PIPE_GCM_H2D_SLICE_STREAMS, default 1)")
    ap.add_argument("--stripe", action="store_true",
                    help="stripe each causal group over the slice streams as the reference does")
    ap.add_argument("--verify-before-release", action="store_true",
                    help="reload with SI_RELOAD_VERIFY_BEFORE_RELEASE (tags checked before any plaintext is written)")
    ap.add_argument("--single", action="store_true",
                    help="the headline workload only (by default its run also times every other workload)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC byte calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: records are independent and need no exchange; "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import secure_infer_amd as si

    if args.copy_mb:
        n = args.copy_mb << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)  # warm-up: page-table entries of both buffers
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(4):
            dst.copy_(src)
        t1.record()
        torch.cuda.synchronize()
        dt = t0.elapsed_time(t1) * 1e-3 / 4
        # read + write bytes per copy over its time: the device's practical
        # streaming rate, the ceiling of the memory-bound codec kernels
        print(json.dumps({"copy_bytes": n, "launches": 5,
                          "copy_read_plus_write_GB_s": round(2 * n / dt / 1e9, 1)}), flush=True)
        return

    with Range(f"workload:{args.config}"):
        res = run_workload(args.config, args, torch, si, args.steps, args.warmup, not args.no_cpu,
                           args.cpu_budget, args.e2e_steps)
    print(f"[bench] {args.config}: {res['us_per_layer']} us/layer", file=sys.stderr, flush=True)
    if args.config == DEFAULT and not args.single:
        # The other workloads in the same run, so one driver run times all of
        # them: same device measurement and checks, a short CPU leg, no
        # end-to-end leg.  `value` and `config` stay the headline's.
        others = {}
        for name in sorted(CONFIGS):
            if name == DEFAULT:
                continue
            with Range(f"workload:{name}"):
                r = run_workload(name, args, torch, si, min(args.steps, 10), min(args.warmup, 2), not args.no_cpu,
                                 min(args.cpu_budget, 2.0), 0)
            print(f"[bench] {name}: {r['us_per_layer']} us/layer", file=sys.stderr, flush=True)
            others[name] = {k: r[k] for k in ("us_per_layer", "value", "hbm_frac", "ms_per_step", "steps", "warmup",
                                              "bit_exact", "bit_exact_checked", "tamper_fail_closed",
                                              "failed_records_per_step")}
            others[name]["GB_s"] = others[name].pop("value")
            others[name]["config"] = r["config"]
            others[name]["roofline"] = {k: r["roofline"][k] for k in ("achieved", "frac", "kernel_us", "traffic")}
            if "cpu_baseline" in r:
                others[name]["cpu_baseline"] = {k: r["cpu_baseline"][k] for k in ("value", "unit", "cores",
                                                                                  "us_per_layer", "matches_gpu")}
            torch.cuda.empty_cache()
        res["other_workloads"] = others
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
