"""Benchmark of the paged decode-attention hot path on one MI355X.

Workload (one "step"): store_kvcache of the batch's new token (64 rows) and
paged GQA decode attention at Qwen3-8B geometry -- 32 query heads, 8 KV
heads, head_dim 128, bf16, block size 256, batch 64, context lengths
U[2048, 8192], a 4096-block K/V pool with values N(0,1). Three independent
random block assignments of the same lengths are rotated across steps so the
256 MB last-level cache cannot serve repeats. Inputs are resident in HBM
before timing starts.

Printed JSON line: decode GB/s (algorithmic K/V/q/out/table bytes over the
decode time), the roofline of the dominant kernel (split-K decode) with its
HIP-event duration, the compression step time at batch 500 (top-20, window
4 blocks, keep 513), varlen causal prefill over the paged cache at Qwen3-8B
geometry (16 prompts U[512,4096], and 2048-token chunks after prefixes
U[0,8192]) in TFLOP/s against the bf16 MFMA peak, the store_kvcache rate of
the prefill-sized scatter, and the oracle's CPU decode rate on a bounded
sample.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
nkv = importlib.import_module("nanokv-llm_amd")
_lib = importlib.import_module("nanokv-llm_amd._lib")
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged decode-attn GB/s (% HBM peak) @Qwen3-8B; KV-compress step µs @bs500"
# the dominant kernel of the decode workload (the roofline line), as rocprofv3 names it
DECODE_KERNEL = "paged_decode_split_kernel<false, 2, 128, false>"
DECODE_PROFILE = "paged_decode_qwen3_8b_bs64.txt"


def measured_traffic(profile, kernel):
    """HBM bytes per launch of `kernel`, as recorded by the rocprofv3 byte-counter
    runs summarised in profiles/<profile> (None if absent)."""
    path = os.path.join(ROOT, "profiles", profile)
    key = f"traffic_bytes_per_launch {kernel}:"
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--compress-reps", type=int, default=30)
    p.add_argument("--prefill-reps", type=int, default=20)
    p.add_argument("--longctx-steps", type=int, default=10)
    p.add_argument("--only", choices=["all", "decode", "compress", "prefill", "longctx",
                                      "qkrope", "metadata"],
                   default="all",
                   help="run one part only (for profiling)")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="also run 5 device-to-device copies of this many MiB (a kernel of "
                        "known traffic, to scale hardware byte counters)")
    return p.parse_args()


def copy_calibration(mib, dev):
    """Five plain copies of `mib` MiB: reads and writes exactly mib MiB each."""
    src = torch.empty(mib * 1024 * 1024, dtype=torch.uint8, device=dev).fill_(3)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] copy calibration: 5 x {mib} MiB device copies", file=sys.stderr, flush=True)


def decode_setup(dev):
    wl = wl_mod.decode_qwen3_8b(seed=2, device=dev, n_table_sets=3)
    sets = []
    width = max(t.size(1) for t in wl["block_tables"])
    for bt, slots in zip(wl["block_tables"], wl["slot_mappings"]):
        btp = torch.full((bt.size(0), width), -1, dtype=torch.int32)
        btp[:, :bt.size(1)] = bt
        sets.append((btp.to(dev), slots.to(dev)))
    return wl, sets


def run_decode(args, dev):
    wl, sets = decode_setup(dev)
    q, key, value = wl["q"].to(dev), wl["key"].to(dev), wl["value"].to(dev)
    kc, vc = wl["k_cache"], wl["v_cache"]
    ctx = wl["context_lens"].to(dev)
    bs, Hq, D = q.shape
    NB, B, Hk, _ = kc.shape
    width = sets[0][0].size(1)
    lib = _lib.lib()
    ws = torch.empty(lib.nkv_paged_decode_workspace_bytes(bs, Hq, D, width, B), dtype=torch.uint8,
                     device=dev)
    out = torch.empty(bs, Hq, D, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream

    def step(i, ev=None):
        bt, slots = sets[i % len(sets)]
        if ev:
            ev[0].record(stream)
        nkv.store_kvcache(key, value, kc, vc, slots)
        if ev:
            ev[1].record(stream)
        _lib.check(lib.nkv_paged_decode_split(q.data_ptr(), q.stride(0), kc.data_ptr(),
                                              vc.data_ptr(), bt.data_ptr(), bt.stride(0),
                                              ctx.data_ptr(), bs, Hq, Hk, D, B, width, NB,
                                              wl["scale"], ws.data_ptr(), ws.numel(), sh),
                   "split")
        if ev:
            ev[2].record(stream)
        _lib.check(lib.nkv_paged_decode_combine(ctx.data_ptr(), bs, Hq, Hk, D, B, width,
                                                out.data_ptr(), out.stride(0), ws.data_ptr(),
                                                ws.numel(), sh), "combine")
        if ev:
            ev[3].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the timed steps hold only the step's own launches; the per-kernel breakdown comes
    # from a second pass with events between the kernels
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    split_ms = [e[1].elapsed_time(e[2]) for e in evs]
    dec_ms = [e[1].elapsed_time(e[3]) for e in evs]
    store_ms = [e[0].elapsed_time(e[1]) for e in evs]
    dec_bytes = wl_mod.decode_bytes(wl["context_lens"], Hq, Hk, D, width)
    split_bytes = dec_bytes - bs * Hq * D * 2  # the combine writes the output
    res = dict(
        ms_per_step=total_ms / args.steps,
        decode_ms=statistics.mean(dec_ms),
        split_ms=statistics.mean(split_ms),
        store_ms=statistics.mean(store_ms),
        decode_bytes=dec_bytes,
        split_bytes=split_bytes,
    )
    # parity spot check of the last step's output against the oracle (4 sequences)
    res["parity_max_abs_err"] = parity_sample(wl, sets[(args.steps - 1) % len(sets)][0], out, kc,
                                              vc, n=4)
    return wl, sets, res


def run_decode_fp8(args, dev, wl, sets):
    """The same decode workload over an fp8 (E4M3FN, scales 1) copy of the pool: store_fp8 +
    decode_fp8 per step on the rotated tables; half the cache bytes per decoded token."""
    kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")
    q, key, value = wl["q"].to(dev), wl["key"].to(dev), wl["value"].to(dev)
    kq, vq = kvc.fp8_quantize(wl["k_cache"]), kvc.fp8_quantize(wl["v_cache"])
    ctx = wl["context_lens"].to(dev)
    bs, Hq, D = q.shape
    NB, B, Hk, _ = kq.shape
    width = sets[0][0].size(1)
    ws = torch.empty(_lib.lib().nkv_paged_decode_workspace_bytes(bs, Hq, D, width, B),
                     dtype=torch.uint8, device=dev)
    out = torch.empty(bs, Hq, D, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream()

    def step(i, ev=None):
        bt, slots = sets[i % len(sets)]
        nkv.store_kvcache(key, value, kq, vq, slots)
        if ev:
            ev[0].record(stream)
        nkv.paged_decode(q, kq, vq, ctx, bt, wl["scale"], out=out, workspace=ws)
        if ev:
            ev[1].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    dec_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    n_tok = int(wl["context_lens"].sum())
    nbytes = n_tok * Hk * D * 2 + bs * Hq * D * 2 * 2 + bs * 4 * (width + 1)
    kd, vd = kvc.fp8_dequantize(kq), kvc.fp8_dequantize(vq)
    err = parity_sample(wl, sets[(args.steps - 1) % len(sets)][0], out, kd, vd, n=4)
    del kq, vq, kd, vd, ws
    torch.cuda.empty_cache()
    return {"decode_fp8_us": round(dec_ms * 1e3, 2),
            "decode_fp8_gbs": round(nbytes / (dec_ms * 1e-3) / 1e9, 1),
            "decode_fp8_bytes": nbytes,
            "decode_fp8_parity_max_abs_err": err}


def _gather_sample(wl, bt, kc, vc, n):
    """Copy the blocks of the first n sequences to host: compact pool + remapped table."""
    return _gather_sample_rows(bt[:n].cpu(), kc, vc)


def parity_sample(wl, bt, out, kc, vc, n):
    from oracle.attention_ref import paged_decode_ref
    kh, vh, bt2 = _gather_sample(wl, bt, kc, vc, n)
    ref = paged_decode_ref(wl["q"][:n].float(), kh, vh, wl["context_lens"][:n], bt2,
                           wl["scale"])
    return float((out[:n].float().cpu() - ref).abs().max())


def cpu_baseline(wl, bt, kc, vc, budget_s=12.0):
    """The oracle's fp32 paged decode (PyTorch on host cores) on a bounded sample."""
    from oracle.attention_ref import paged_decode_ref
    n = 16
    kh, vh, bt2 = _gather_sample(wl, bt, kc, vc, n)
    q = wl["q"][:n].float()
    ctx = wl["context_lens"][:n]
    nbytes = wl_mod.decode_bytes(ctx, q.size(1), kh.size(2), 128, bt2.size(1))
    times = []
    t_end = time.perf_counter() + budget_s
    paged_decode_ref(q, kh, vh, ctx, bt2, wl["scale"])  # warm-up
    while time.perf_counter() < t_end or len(times) < 2:
        t = time.perf_counter()
        paged_decode_ref(q, kh, vh, ctx, bt2, wl["scale"])
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle paged_decode_ref (fp32 torch CPU) on 16 of the 64 sequences "
                      f"({int(ctx.sum())} tokens, {nbytes / 1e6:.0f} MB), median of "
                      f"{len(times)} runs; host has {os.cpu_count()} logical CPUs"}


def compress_parity(q, kg, vg, bt, lens, sel, agg, dev):
    """The last layer's compression step (compress_step with the finalize's table, slot and
    event update in the same launch) once on a device copy of the selected sequences' blocks, against the oracle on a
    host copy of the same blocks: importance within rtol 1e-4 (max relative error reported),
    kept sets exact given the scores, caches, lengths, events, tables and slots bit-exact. The
    timed state is left untouched, so this works on a pool that fills most of HBM."""
    from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                     get_tail_window_and_tail_slots_ref, select_topk_ref,
                                     snapkv_importance_ref)
    bt, lens = bt.cpu(), lens.cpu()
    ids = sorted({int(x) for x in bt[sel].flatten().tolist() if x >= 0})
    remap = {b: j for j, b in enumerate(ids)}
    bt2 = torch.full_like(bt, -1)
    for i in sel:
        bt2[i] = torch.tensor([remap.get(int(x), -1) for x in bt[i].tolist()], dtype=torch.int32)
    idx = torch.tensor(ids, device=dev)
    kc, vc = kg.index_select(0, idx), vg.index_select(0, idx)
    kh, vh = kc.cpu(), vc.cpu()
    bs, Hq, D = q.shape
    B = kg.size(1)
    btg, base = bt2.to(dev), lens.to(dev)
    ctx = base.clone()
    seq_idx = torch.tensor(sel, dtype=torch.int32, device=dev)
    slot_map = torch.arange(bs, dtype=torch.int32, device=dev) * 3
    events = torch.empty(len(sel), 4 + bt.size(1), dtype=torch.int32, device=dev)
    keep, imp = cu.compress_step(q, kc, vc, btg, base, ctx, seq_idx, 4, 513, D ** -0.5, agg,
                                 events=events, rewrite_tables=True, slot_mapping=slot_map)
    torch.cuda.synchronize()
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(bt2, lens, st, B, 4)
    k_sub, _ = gather_kv_by_slots_ref(kh, vh, slots)
    ref_imp = snapkv_importance_ref(q.cpu().index_select(0, st).unsqueeze(2), k_sub, 1, "fp32",
                                    agg)
    imp = imp.cpu()
    rel = float(((imp - ref_imp).abs() / ref_imp.abs().clamp(min=1e-7)).max())
    keep = keep.cpu().long()
    kept_exact = bool(torch.equal(keep[..., 1:-1], select_topk_ref(imp, 511)))
    ctx_ref = lens.clone()
    _, _, ev_ref = compress_compact_ref(None, kh, vh, bt2, lens, ctx_ref, sel, B, 4, 2, 1, 0, 1,
                                        keep_idx=keep)
    caches = bool(torch.equal(kc.cpu(), kh) and torch.equal(vc.cpu(), vh))
    bt_exp, slot_exp = bt2.clone(), torch.arange(bs, dtype=torch.int32) * 3
    for ev in ev_ref:
        i, n = ev["batch_index"], ev["new_context_len"]
        bt_exp[i, ev["keep_blocks"]:] = -1
        slot_exp[i] = -1 if n % B == 0 else int(bt2[i, n // B]) * B + n % B
    meta = bool(torch.equal(ctx.cpu(), ctx_ref) and cu.events_to_dicts(events, 0) == ev_ref
                and torch.equal(btg.cpu(), bt_exp) and torch.equal(slot_map.cpu(), slot_exp))
    del kc, vc
    return {"importance_max_rel_err": rel, "importance_within_1e-4": rel <= 1e-4,
            "kept_sets_exact_given_scores": kept_exact, "caches_bit_exact": caches,
            "lengths_events_tables_slots_exact": meta}


def compress_in_graph(args, dev, flush, n_in=10):
    """The full step inside a larger graph, as it runs in a decode step's graph (whose own
    launch is paid once for the whole step): n_in steps captured in one graph, per step. The
    state is the whole batch-500 decode state (every sequence's blocks in the pool); step i
    compresses its own 20 sequences, ranks 20i .. 20i+19 by length (step 0: the 20 longest,
    the configuration's selection), so every step reads cold windows, and has its own copy
    of the tables (restored outside the timed region)."""
    cw = wl_mod.compress_workload(500, 32, 8, 1500, 4096, 20, 3, dev, selected_only=False)
    kg, vg, q = cw["k_cache"], cw["v_cache"], cw["q"].to(dev)
    lens = cw["context_lens"].tolist()
    order = sorted(range(len(lens)), key=lambda i: (-lens[i], i))
    sels = [torch.tensor(sorted(order[20 * i:20 * i + 20]), dtype=torch.int32, device=dev)
            for i in range(n_in)]
    bt0 = cw["block_tables"].to(dev)
    bts = [bt0.clone() for _ in range(n_in)]
    base = cw["context_lens"].to(dev)
    ctx = base.clone()
    Hq, Hk = q.size(1), kg.size(2)
    ws = torch.empty(cu.select_workspace_bytes(20, Hq, Hk, 4, 256), dtype=torch.uint8,
                     device=dev)
    events = torch.empty(20, 4 + bt0.size(1), dtype=torch.int32, device=dev)
    slot_map = torch.zeros(base.numel(), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    res = {}
    for agg in ("group", "all"):
        n_sets = 1 if agg == "all" else Hk
        imp = torch.empty(20, n_sets, 1023, dtype=torch.float32, device=dev)
        keep = torch.empty(20, n_sets, 513, dtype=torch.int32, device=dev)

        def steps():
            for sel, btx in zip(sels, bts):
                cu.compress_step(q, kg, vg, btx, base, ctx, sel, 4, 513, 128 ** -0.5, agg,
                                 importance=imp, keep_idx=keep, workspace=ws, events=events,
                                 rewrite_tables=True, slot_mapping=slot_map)

        steps()  # every kernel loaded before the capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            steps()
        times = []
        for i in range(3 + args.compress_reps):
            for btx in bts:
                btx.copy_(bt0)
            flush.sum()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            graph.replay()
            b.record(stream)
            torch.cuda.synchronize()
            if i >= 3:
                times.append(a.elapsed_time(b) * 1000.0 / n_in)
        del graph
        key = "compress_step_in_graph_us" if agg == "group" else "compress_step_all_in_graph_us"
        res[key] = round(statistics.median(times), 2)
    del kg, vg, cw
    torch.cuda.empty_cache()
    return res


def run_compress(args, dev):
    """One layer's compression step at batch 500 as the configuration states it: scoring,
    top-k and compaction of the 20 longest sequences (window 4 blocks, keep 513), and the
    block-table, slot-mapping and event update, in one launch (the last layer's step), per
    KV head (agg "group", the benchmark configuration) and with the reference's all-head
    importance (agg "all"). compress_select_compact_us: the step without the update;
    compress_step_two_launch_us: the update as compress_finalize's own launch."""
    cw = wl_mod.compress_qwen3_8b(seed=3, device=dev, selected_only=True)
    kg, vg = cw["k_cache"], cw["v_cache"]
    bt0 = cw["block_tables"].to(dev)
    btg, base = bt0.clone(), cw["context_lens"].to(dev)
    ctx = base.clone()
    sel = torch.tensor(cw["seq_idx"], dtype=torch.int32, device=dev)
    q = cw["q"].to(dev)
    m = sel.numel()
    Hq, Hk = q.size(1), kg.size(2)
    wsb = cu.select_workspace_bytes(m, Hq, Hk, 4, 256)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    events = torch.empty(m, 4 + btg.size(1), dtype=torch.int32, device=dev)
    slot_map = torch.zeros(base.numel(), dtype=torch.int32, device=dev)
    flush = torch.ones(128 * 1024 * 1024, dtype=torch.int32, device=dev)  # 512 MiB
    stream = torch.cuda.current_stream()
    lens = cw["context_lens"][cw["seq_idx"]].to(torch.int64)
    tails = lens % 256
    nbytes = m * 1024 * 2048 + m * Hq * 128 * 2 + 2 * int((513 + tails).sum()) * 4096
    res = {f"compress_parity_{agg}": compress_parity(q, kg, vg, cw["block_tables"],
                                                     cw["context_lens"], cw["seq_idx"], agg, dev)
           for agg in ("group", "all")}

    def timed_many(fns, reps):
        """Median µs of each variant; the variants' reps interleave (order reversed every
        other round) so that a drift of the clock over the run weighs on all alike."""
        times = {n: [] for n in fns}
        order = list(fns)
        for i in range(3 + reps):
            for n in (order if i % 2 == 0 else order[::-1]):
                btg.copy_(bt0)  # the finalize's table rewrite is undone outside the timed region
                # evict the window from the 256 MB last-level cache by READING 512 MiB: the
                # cache is left holding clean lines, as after the decode kernels that run
                # between compression steps (a fill would leave 256 MB of dirty lines
                # whose write-back would overlap the step)
                flush.sum()
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                fns[n]()
                b.record(stream)
                torch.cuda.synchronize()
                if i >= 3:
                    times[n].append(a.elapsed_time(b) * 1000.0)
        return {n: statistics.median(t) for n, t in times.items()}

    def timed(fn, reps):
        return timed_many({"": fn}, reps)[""]

    for agg in ("group", "all"):
        n_sets = 1 if agg == "all" else Hk
        imp = torch.empty(m, n_sets, 1023, dtype=torch.float32, device=dev)
        keep = torch.empty(m, n_sets, 513, dtype=torch.int32, device=dev)

        def step():
            cu.compress_step(q, kg, vg, btg, base, ctx, sel, 4, 513, 128 ** -0.5, agg,
                             importance=imp, keep_idx=keep, workspace=ws)

        def full_step():
            cu.compress_step(q, kg, vg, btg, base, ctx, sel, 4, 513, 128 ** -0.5, agg,
                             importance=imp, keep_idx=keep, workspace=ws, events=events,
                             rewrite_tables=True, slot_mapping=slot_map)

        def two_launches():
            step()
            cu.compress_finalize(btg, base, sel, 513, 256, 4, events, rewrite_tables=True,
                                 slot_mapping=slot_map)

        variants = {"full": full_step, "step": step}
        if agg == "group":
            variants["two"] = two_launches
        t = timed_many(variants, args.compress_reps)
        med = t["full"]
        key = "compress_step_us" if agg == "group" else "compress_step_all_us"
        res[key] = round(med, 2)
        res[key.replace("_us", "_gbs")] = round(nbytes / (med * 1e-6) / 1e9, 1)
        key2 = "compress_select_compact_us" if agg == "group" else "compress_select_compact_all_us"
        res[key2] = round(t["step"], 2)
        if agg == "group":
            res["compress_step_two_launch_us"] = round(t["two"], 2)
    # the same step over an fp8 (E4M3FN) copy of the pool (agg "group")
    kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")
    kq, vq = kvc.fp8_quantize(kg), kvc.fp8_quantize(vg)
    imp = torch.empty(m, Hk, 1023, dtype=torch.float32, device=dev)
    keep = torch.empty(m, Hk, 513, dtype=torch.int32, device=dev)
    res["compress_step_fp8_us"] = round(timed(lambda: cu.compress_step(
        q, kq, vq, btg, base, ctx, sel, 4, 513, 128 ** -0.5, "group", importance=imp,
        keep_idx=keep, workspace=ws, events=events, rewrite_tables=True,
        slot_mapping=slot_map), args.compress_reps), 2)
    del kq, vq
    res.update(compress_in_graph(args, dev, flush))
    if not args.no_cpu_baseline:
        res["compress_cpu_baseline"] = cpu_compress_baseline()
    res.update({"compress_bytes": nbytes, "compress_sequences": m,
                "compress_config": "the full step (select + compact + the finalize's tables, "
                                   "slots and events, one launch); agg group (importance "
                                   "summed over each GQA group, kept set per KV head); "
                                   "compress_step_all_*: all-head importance; "
                                   "compress_select_compact_*: without the finalize; "
                                   "compress_step_two_launch_us: the finalize as its own "
                                   "launch; compress_step_fp8_us: the full step, agg group, "
                                   "over an fp8 pool; *_in_graph_us: per step, ten full "
                                   "steps of the whole batch-500 state in one graph, each "
                                   "on its own 20 sequences (the 20 longest, then the next "
                                   "ranks; cold windows)"})
    return res


def cpu_compress_baseline(n_sample=4, budget_s=6.0):
    """The oracle's compression step (the reference's chain: gather the window, bf16 SnapKV
    scores, top-k, two-phase compaction) on the host cores, for n_sample of the 20 selected
    sequences of the batch-500 state, scaled to the 20-sequence step."""
    from oracle.compress_ref import compress_compact_ref
    cw = wl_mod.compress_qwen3_8b(seed=3, device="cpu", selected_only=True)
    sel = cw["seq_idx"][:n_sample]
    kc, vc = cw["k_cache"], cw["v_cache"]
    ts, t_end = [], time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(ts) < 2:
        ctx = cw["context_lens"].clone()
        t = time.perf_counter()
        compress_compact_ref(cw["q"], kc, vc, cw["block_tables"], cw["context_lens"], ctx, sel,
                             256, 4, 2, 1, 0, 1, score_dtype="bf16", agg="group")
        ts.append(time.perf_counter() - t)
    per_step = statistics.median(ts) * len(cw["seq_idx"]) / n_sample
    return {"value": round(per_step * 1e6, 1), "unit": "us per step",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle compress_compact_ref (torch CPU, bf16 scores, agg group) on "
                      f"{n_sample} of the {len(cw['seq_idx'])} selected sequences, median of "
                      f"{len(ts)} runs, scaled x{len(cw['seq_idx']) / n_sample:g}"}


def prefill_flops(Lq, Lk, Hq, D=128):
    """4*Hq*D per visible (query, key) pair; query j of a sequence sees Lk-Lq+j+1 keys."""
    pairs = sum(q * (k - q) + q * (q + 1) // 2 for q, k in zip(Lq, Lk))
    return 4 * Hq * D * pairs


def run_prefill_one(args, dev, name, wl):
    """store_kvcache of the prompt rows, then varlen causal prefill over the paged cache."""
    kc, vc = wl["k_cache"], wl["v_cache"]
    key, value, slots = wl["key"], wl["value"], wl["slot_mapping"].to(dev)
    q = wl["q"]
    cq, ck = wl["cu_seqlens_q"].to(dev), wl["cu_seqlens_k"].to(dev)
    bt = wl["block_tables"].to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()

    def ev():
        return torch.cuda.Event(enable_timing=True)

    store_t, pre_t = [], []
    for i in range(3 + args.prefill_reps):
        e0, e1, e2 = ev(), ev(), ev()
        e0.record(stream)
        nkv.store_kvcache(key, value, kc, vc, slots)
        e1.record(stream)
        nkv.varlen_prefill(q, kc, vc, cq, ck, wl["max_seqlen_q"], wl["scale"], block_tables=bt,
                           out=out)
        e2.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            store_t.append(e0.elapsed_time(e1))
            pre_t.append(e1.elapsed_time(e2))
    flops = prefill_flops(wl["Lq"], wl["Lk"], wl["Hq"])
    pre_ms = statistics.median(pre_t)
    st_ms = statistics.median(store_t)
    n_rows = key.size(0)
    st_bytes = 2 * 2 * n_rows * key.size(1) * key.size(2) * 2 + n_rows * 4  # K,V read+write
    tflops = flops / (pre_ms * 1e-3) / 1e12
    # parity: the last min(128, Lq) queries of the shortest sequence vs the oracle
    from oracle.attention_ref import varlen_prefill_ref
    i = min(range(len(wl["Lq"])), key=lambda j: wl["Lq"][j])
    Lq_i, Lk_i = wl["Lq"][i], wl["Lk"][i]
    nq = min(128, Lq_i)
    r0 = int(wl["cu_seqlens_q"][i]) + Lq_i - nq
    btr = wl["block_tables"][i:i + 1]
    kh, vh, bt2 = _gather_sample_rows(btr, kc, vc)
    ref = varlen_prefill_ref(q[r0:r0 + nq].float().cpu(), kh, vh,
                             torch.tensor([0, nq], dtype=torch.int32),
                             torch.tensor([0, Lk_i], dtype=torch.int32), wl["scale"],
                             block_tables=bt2)
    err = float((out[r0:r0 + nq].float().cpu() - ref).abs().max())
    extra = {}
    if not args.no_cpu_baseline:
        # the same oracle call timed on the host cores: the reference path's cost per flop
        args_ref = (q[r0:r0 + nq].float().cpu(), kh, vh, torch.tensor([0, nq], dtype=torch.int32),
                    torch.tensor([0, Lk_i], dtype=torch.int32), wl["scale"])
        ts, t_end = [], time.perf_counter() + 6.0
        while time.perf_counter() < t_end or len(ts) < 2:
            t = time.perf_counter()
            varlen_prefill_ref(*args_ref, block_tables=bt2)
            ts.append(time.perf_counter() - t)
        f_s = prefill_flops([nq], [Lk_i], wl["Hq"])
        extra[f"{name}_cpu_baseline"] = {
            "value": round(f_s / statistics.median(ts) / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle varlen_prefill_ref (fp32 torch CPU): the last {nq} queries of "
                      f"one sequence over {Lk_i} paged keys ({f_s / 1e9:.1f} GFLOP), median "
                      f"of {len(ts)} runs"}
    return {
        **extra,
        f"{name}_us": round(pre_ms * 1e3, 1),
        f"{name}_tflops": round(tflops, 1),
        f"{name}_pct_mfma_peak": round(100.0 * tflops / MFMA_BF16_PEAK_TFLOPS, 1),
        f"{name}_gflop": round(flops / 1e9, 1),
        f"{name}_parity_max_abs_err": err,
        f"{name}_store_us": round(st_ms * 1e3, 1),
        f"{name}_store_gbs": round(st_bytes / (st_ms * 1e-3) / 1e9, 1),
    }


def _gather_sample_rows(btr, kc, vc):
    """Blocks of the given table rows copied to host, with the table remapped."""
    ids = sorted({int(x) for x in btr.flatten().tolist() if x >= 0})
    remap = {b: j for j, b in enumerate(ids)}
    idx = torch.tensor(ids, device=kc.device)
    kh, vh = kc.index_select(0, idx).cpu(), vc.index_select(0, idx).cpu()
    bt2 = torch.tensor([[remap.get(int(x), -1) for x in row] for row in btr.tolist()],
                       dtype=torch.int32)
    return kh, vh, bt2


def run_prefill_fp8(args, dev):
    """Chunked prefill reading an fp8 (E4M3FN) pool in place: the prefill kernel's fp8
    instance widens the codes while it stages each K/V tile."""
    kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")
    wl = wl_mod.prefill_chunked_qwen3_8b(device=dev)
    kq, vq = kvc.fp8_quantize(wl["k_cache"]), kvc.fp8_quantize(wl["v_cache"])
    del wl["k_cache"], wl["v_cache"]
    q = wl["q"]
    cq, ck = wl["cu_seqlens_q"].to(dev), wl["cu_seqlens_k"].to(dev)
    bt = wl["block_tables"].to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()
    t = []
    for i in range(3 + args.prefill_reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        nkv.varlen_prefill(q, kq, vq, cq, ck, wl["max_seqlen_q"], wl["scale"], block_tables=bt,
                           out=out, max_seqlen_k=wl["max_seqlen_k"])
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            t.append(a.elapsed_time(b))
    ms = statistics.median(t)
    flops = prefill_flops(wl["Lq"], wl["Lk"], wl["Hq"])
    del kq, vq, out
    torch.cuda.empty_cache()
    return {"prefill_chunked_fp8_us": round(ms * 1e3, 1),
            "prefill_chunked_fp8_tflops": round(flops / (ms * 1e-3) / 1e12, 1)}


def run_prefill(args, dev):
    res = {}
    for name, fn in (("prefill", wl_mod.prefill_qwen3_8b),
                     ("prefill_chunked", wl_mod.prefill_chunked_qwen3_8b)):
        wl = fn(device=dev)
        res.update(run_prefill_one(args, dev, name, wl))
        del wl
        torch.cuda.empty_cache()
    res.update(run_prefill_fp8(args, dev))
    return res


def qkrope_bytes(n_tokens, Hq, Hk, need_k, D=128):
    """Algorithmic HBM bytes of one fused norm + rope + store: read the q/k/v head rows,
    position, slot and cos|sin row; write q', the K and V cache rows (and k' if asked)."""
    per_tok = (Hq + 2 * Hk) * D * 2 + 8 + 4 + D * 4 + (Hq + 2 * Hk + (Hk if need_k else 0)) * D * 2
    return n_tokens * per_tok


def _qkrope_unfused(pos, q, k, v, cs, qw, kw, kc, vc, slots):
    """The reference's sequence of separate passes (layernorm.py:21-26 twice,
    rotary_embedding.py:7-15 twice, then store_kvcache) as eager torch ops on the GPU,
    timed only to show what the fusion saves."""
    def norm(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype) * w

    def rope(x, c, s_):
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        return torch.cat((x1 * c - x2 * s_, x2 * c + x1 * s_), dim=-1).to(x.dtype)

    c, s_ = cs[pos].unsqueeze(1).chunk(2, dim=-1)
    q2, k2 = rope(norm(q, qw), c, s_), rope(norm(k, kw), c, s_)
    nkv.store_kvcache(k2, v, kc, vc, slots)
    return q2, k2


def _graph_call_ms(fn, n_inner=10, reps=20):
    """Per-call GPU time of fn() from a HIP graph holding n_inner back-to-back calls
    (replayed reps times, median): the host's launch latency is not in it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n_inner):
            fn()
    stream = torch.cuda.current_stream()
    t = []
    for i in range(3 + reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            t.append(e0.elapsed_time(e1) / n_inner)
    return statistics.median(t), g


def run_qkrope(args, dev):
    """Fused q/k RMSNorm + RoPE + K/V store at Qwen3-8B geometry (Hq 32, Hk 8): the 16-prompt
    prefill batch (positions 0..L-1, k' also written for the contiguous prefill) and a
    64-token decode batch (k' only into the cache). The fused op is timed inside a replayed
    HIP graph; the unfused eager sequence (launch latency included) is shown beside it."""
    wl = wl_mod.prefill_qwen3_8b(device=dev)
    N, Hq, Hk, D = wl["q"].size(0), 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(9)
    qkv = torch.randn(N, (Hq + 2 * Hk) * D, device=dev, generator=g).to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(N, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hk) * D].view(N, Hk, D)
    v = qkv[:, (Hq + Hk) * D:].view(N, Hk, D)
    qw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    rope = nkv.RotaryEmbedding(D, D, 40960, 1e6, device=dev)
    cs = rope.cos_sin_cache
    kc, vc = wl["k_cache"], wl["v_cache"]
    pos, slots = wl["positions"], wl["slot_mapping"].to(dev)
    q_out = torch.empty(N, Hq, D, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream()
    res = {}
    for name, n, need_k in (("qkrope_prefill", N, True), ("qkrope_decode", 64, False)):
        sl = slice(0, n)
        fused = lambda: nkv.qk_norm_rope_store(pos[sl], q[sl], k[sl], v[sl], cs, qw, kw,  # noqa
                                               1e-6, k_cache=kc, v_cache=vc,
                                               slot_mapping=slots[sl], need_k=need_k,
                                               q_out=q_out[sl])
        fused()
        torch.cuda.synchronize()
        eager_q = q_out[sl].clone()
        fused_ms, graph = _graph_call_ms(fused, reps=args.prefill_reps)
        torch.cuda.synchronize()
        assert torch.equal(q_out[sl], eager_q), "graph replay differs from the eager call"
        del graph
        t = []
        for i in range(5 + args.prefill_reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            _qkrope_unfused(pos[sl], q[sl], k[sl], v[sl], cs.squeeze(1), qw, kw, kc, vc,
                            slots[sl])
            e1.record(stream)
            torch.cuda.synchronize()
            if i >= 5:
                t.append(e0.elapsed_time(e1))
        nbytes = qkrope_bytes(n, Hq, Hk, need_k)
        res[f"{name}_tokens"] = n
        res[f"{name}_us"] = round(fused_ms * 1e3, 2)
        res[f"{name}_gbs"] = round(nbytes / (fused_ms * 1e-3) / 1e9, 1)
        res[f"{name}_unfused_torch_us"] = round(statistics.median(t) * 1e3, 2)
    res["qkrope_bytes_per_token"] = qkrope_bytes(1, Hq, Hk, True)
    # parity on the first 64 prefill tokens against the oracle
    from oracle.rope_ref import qk_norm_rope_store_ref
    qo, ko, _ = nkv.qk_norm_rope_store(pos[:64], q[:64], k[:64], v[:64], cs, qw, kw, 1e-6)
    qr, kr, _ = qk_norm_rope_store_ref(qkv[:64].cpu(), pos[:64].cpu(), qw.cpu(), kw.cpu(), 1e-6,
                                       cs.squeeze(1).cpu(), Hq, Hk)
    res["qkrope_parity_max_abs_err"] = max(float((qo.float().cpu() - qr.float()).abs().max()),
                                           float((ko.float().cpu() - kr.float()).abs().max()))
    del wl
    torch.cuda.empty_cache()
    return res


def run_metadata(args, dev):
    """Per-step metadata (positions, slot_mapping, cu_seqlens, context_lens, padded block
    tables) for the 16-prompt prefill batch (38,632 tokens) and a batch-500 decode step with
    tables up to 64 blocks: the device builder (host packing + one copy + two kernels,
    synchronised wall time) vs the reference's per-token Python loop (the oracle's
    restatement, moved to the device the way prepare_step does)."""
    from oracle.metadata_ref import prepare_step_ref
    md = importlib.import_module("nanokv-llm_amd.engine.metadata")
    gen = torch.Generator().manual_seed(11)
    wl = wl_mod.prefill_qwen3_8b()  # CPU copy: only lengths and tables are used
    tables_p = [[int(x) for x in row if x >= 0] for row in wl["block_tables"].tolist()]
    cases = {
        "prefill": ([0] * len(wl["Lq"]), list(wl["Lq"]), tables_p, None),
    }
    lens = torch.exp(torch.empty(500).uniform_(6.93, 9.70, generator=gen)).long().tolist()
    perm = torch.randperm(40000, generator=gen).tolist()
    tables_d, o = [], 0
    for n in lens:
        nb = (n + 255) // 256
        tables_d.append(perm[o:o + nb])
        o += nb
    cases["decode"] = ([n - 1 for n in lens], [1] * len(lens), tables_d, [0] * len(lens))
    res = {}
    for name, (starts, num_new, tables, offs) in cases.items():
        def dev_build():
            return md.build_step_metadata(starts, num_new, tables, 256, dev, pos_offsets=offs)

        def ref_build():
            r = prepare_step_ref(starts, num_new, tables, 256, pos_offsets=offs)
            return {k: (v.to(dev, non_blocking=True) if torch.is_tensor(v) else v)
                    for k, v in r.items()}
        t = {}
        for tag, fn in (("device", dev_build), ("cpu_loop", ref_build)):
            ts = []
            for i in range(3 + 10):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                out = fn()
                torch.cuda.synchronize()
                if i >= 3:
                    ts.append(time.perf_counter() - t0)
            t[tag] = statistics.median(ts)
            if tag == "device":
                got = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in out.items()}
        ref = prepare_step_ref(starts, num_new, tables, 256, pos_offsets=offs)
        ok = all(torch.equal(got[k], ref[k]) for k in ("positions", "slot_mapping",
                                                     "cu_seqlens_q", "cu_seqlens_k",
                                                     "context_lens", "block_tables"))
        res[f"metadata_{name}_tokens"] = sum(num_new)
        res[f"metadata_{name}_device_us"] = round(t["device"] * 1e6, 1)
        res[f"metadata_{name}_cpu_loop_us"] = round(t["cpu_loop"] * 1e6, 1)
        res[f"metadata_{name}_bit_exact"] = ok
    # steady-state decode with the device-resident table store: per step ~2 of the 500
    # tables gain a block (one block per 256 tokens per sequence)
    starts, num_new, tables, offs = cases["decode"]
    tables = [list(t) for t in tables]
    store = md.BlockTableStore(512, 128, dev)
    ids = list(range(len(tables)))
    md.build_step_metadata(starts, num_new, tables, 256, dev, pos_offsets=offs, store=store,
                           seq_ids=ids)
    ts, nxt = [], 50000
    for i in range(3 + 20):
        for j in (i % 500, (i * 37 + 11) % 500):
            tables[j].append(nxt)
            nxt += 1
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = md.build_step_metadata(starts, num_new, tables, 256, dev, pos_offsets=offs,
                                     store=store, seq_ids=ids)
        torch.cuda.synchronize()
        if i >= 3:
            ts.append(time.perf_counter() - t0)
    ref = prepare_step_ref(starts, num_new, tables, 256, pos_offsets=offs)
    res["metadata_decode_store_us"] = round(statistics.median(ts) * 1e6, 1)
    res["metadata_decode_store_bit_exact"] = all(
        torch.equal(out[k].cpu(), ref[k]) for k in ("positions", "slot_mapping", "block_tables",
                                                    "context_lens"))
    return res


def run_longctx(args, dev):
    """Qwen3-32B long-context decode at batch 500 on a pool filling most of HBM, and the
    compression step on that state (20 longest uncompressed sequences, window 4 blocks, keep
    513, agg "group"), amortised over its 1024-step period; the same step with the selection
    made on the device and the events written, replayed from a HIP graph."""
    torch.cuda.empty_cache()
    wl = wl_mod.decode_qwen3_32b_longctx(seed=6, device=dev)
    kc, vc = wl["k_cache"], wl["v_cache"]
    bt, slots = wl["block_tables"][0].to(dev), wl["slot_mappings"][0].to(dev)
    q, key, value = wl["q"].to(dev), wl["key"].to(dev), wl["value"].to(dev)
    ctx = wl["context_lens"].to(dev)
    bs, Hq, D = q.shape
    NB, B, Hk, _ = kc.shape
    width = bt.size(1)
    lib = _lib.lib()
    ws = torch.empty(lib.nkv_paged_decode_workspace_bytes(bs, Hq, D, width, B), dtype=torch.uint8,
                     device=dev)
    out = torch.empty(bs, Hq, D, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream()

    def step():
        nkv.store_kvcache(key, value, kc, vc, slots)
        nkv.paged_decode(q, kc, vc, ctx, bt, wl["scale"], out=out, workspace=ws)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.longctx_steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / args.longctx_steps
    nbytes = wl_mod.decode_bytes(wl["context_lens"], Hq, Hk, D, width)
    parity = parity_sample(wl, bt, out, kc, vc, n=4)
    # compression: the 20 longest sequences eligible under the engine's rule, checked against
    # the oracle on a copy of their blocks, then timed as the full step (select + compact +
    # table, slot and event update; the table rewrite undone outside the timed region)
    sel_list = wl_mod.eligible_longest(wl["context_lens"].tolist(),
                                       wl["tail_uncompressed"].tolist(), 20, B, 4)
    lens = wl["context_lens"].tolist()
    comp_parity = {agg: compress_parity(q, kc, vc, bt, ctx, sel_list, agg, dev)
                   for agg in ("group", "all")}
    sel = torch.tensor(sel_list, dtype=torch.int32, device=dev)
    base = ctx.clone()
    cl = ctx.clone()
    bt_c = bt.clone()
    m = sel.numel()
    cws = torch.empty(cu.select_workspace_bytes(m, Hq, Hk, 4, B), dtype=torch.uint8, device=dev)
    imp = torch.empty(m, Hk, 4 * B - 1, dtype=torch.float32, device=dev)
    keep = torch.empty(m, Hk, 513, dtype=torch.int32, device=dev)
    ev_c = torch.empty(m, 4 + width, dtype=torch.int32, device=dev)
    slot_c = slots.clone()
    flush = torch.ones(128 * 1024 * 1024, dtype=torch.int32, device=dev)
    times = []
    for i in range(3 + args.compress_reps):
        bt_c.copy_(bt)
        flush.sum()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        cu.compress_step(q, kc, vc, bt_c, base, cl, sel, 4, 513, D ** -0.5, "group",
                         importance=imp, keep_idx=keep, workspace=cws, events=ev_c,
                         rewrite_tables=True, slot_mapping=slot_c)
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            times.append(a.elapsed_time(b) * 1000.0)
    comp_us = statistics.median(times)
    # the same step with the selection made on the device (policy "longest", topk 20, -1
    # padded) and the events written, captured in one HIP graph and replayed
    tails_d = wl["tail_uncompressed"].to(device=dev, dtype=torch.int32)
    i32 = dict(dtype=torch.int32, device=dev)
    counter, sel_d, n_sel = torch.zeros(1, **i32), torch.empty(20, **i32), torch.empty(1, **i32)
    base_d = torch.empty(bs, **i32)
    ev = torch.empty(20, 4 + width, **i32)
    imp20 = torch.empty(20, Hk, 4 * B - 1, dtype=torch.float32, device=dev)
    keep20 = torch.empty(20, Hk, 513, dtype=torch.int32, device=dev)
    cws20 = torch.empty(cu.select_workspace_bytes(20, Hq, Hk, 4, B), dtype=torch.uint8,
                        device=dev)

    def device_step():
        cu.compress_schedule(ctx, tails_d, B, 4, 20, 1, counter, sel_d, n_sel, base_d,
                             policy="longest")
        cu.compress_step(q, kc, vc, bt_c, base_d, cl, sel_d, 4, 513, D ** -0.5, "group",
                         importance=imp20, keep_idx=keep20, workspace=cws20, events=ev,
                         rewrite_tables=True, slot_mapping=slot_c)

    bt_c.copy_(bt)
    device_step()
    torch.cuda.synchronize()
    same_selection = sorted(x for x in sel_d.tolist() if x >= 0) == sel_list
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        device_step()
    gtimes = []
    for i in range(3 + args.compress_reps):
        bt_c.copy_(bt)
        flush.sum()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            gtimes.append(a.elapsed_time(b) * 1000.0)
    del graph
    # The same pair of launches inside a larger graph, as in a decode step's graph, whose
    # own launch is paid once for the whole step: ten schedule + step pairs in one graph,
    # per pair. Pair i may only pick from its own 20 of the 200 longest eligible sequences
    # (the tail counts of the others read 0), so every pair reads cold windows, and each
    # pair has its own copy of the tables.
    n_in = 10
    elig = wl_mod.eligible_longest(wl["context_lens"].tolist(),
                                   wl["tail_uncompressed"].tolist(), 20 * n_in, B, 4)
    tails_n, bt_n = [], []
    for i in range(n_in):
        t = torch.zeros(bs, **i32)
        grp = torch.tensor(elig[20 * i:20 * i + 20], device=dev, dtype=torch.long)
        t[grp] = tails_d[grp]
        tails_n.append(t)
        bt_n.append(bt.clone())
    graph_n = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph_n):
        for t, btx in zip(tails_n, bt_n):
            cu.compress_schedule(ctx, t, B, 4, 20, 1, counter, sel_d, n_sel, base_d,
                                 policy="longest")
            cu.compress_step(q, kc, vc, btx, base_d, cl, sel_d, 4, 513, D ** -0.5, "group",
                             importance=imp20, keep_idx=keep20, workspace=cws20, events=ev,
                             rewrite_tables=True, slot_mapping=slot_c)
    ntimes = []
    for i in range(3 + args.compress_reps):
        for btx in bt_n:
            btx.copy_(bt)
        flush.sum()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph_n.replay()
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            ntimes.append(a.elapsed_time(b) * 1000.0 / n_in)
    del graph_n, bt_n
    gbs = nbytes / (step_ms * 1e-3) / 1e9
    res = {
        "longctx_workload": "Qwen3-32B geometry: Hq 64, Hk 8, batch 500, ctx log-uniform "
                            "[1024,16384] (seed 6), 20% compressed once, store + decode per step",
        "longctx_pool_gb": round(2 * NB * B * Hk * D * 2 / 1e9, 1),
        "longctx_tokens": int(sum(lens)),
        "longctx_step_us": round(step_ms * 1e3, 1),
        "longctx_decode_gbs": round(gbs, 1),
        "longctx_pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 1),
        "longctx_parity_max_abs_err": parity,
        "longctx_compress_parity_group": comp_parity["group"],
        "longctx_compress_parity_all": comp_parity["all"],
        "longctx_compress_step_us": round(comp_us, 2),
        "longctx_compress_amortized_us_per_step": round(comp_us / 1024, 3),
        "longctx_compress_graph_us": round(statistics.median(gtimes), 2),
        "longctx_compress_in_graph_us": round(statistics.median(ntimes), 2),
        "longctx_compress_graph_same_selection": same_selection,
    }
    del wl, kc, vc, ws, out
    torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not "
              "supported (the attention path shards by KV head or by sequence with no "
              "collective, see the design notes).", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.copy_calibration_mib:
        copy_calibration(args.copy_calibration_mib, dev)
    if args.only == "compress":
        comp = run_compress(args, dev)
        print(json.dumps(comp), flush=True)
        return
    if args.only == "prefill":
        print(json.dumps(run_prefill(args, dev)), flush=True)
        return
    if args.only == "longctx":
        print(json.dumps(run_longctx(args, dev)), flush=True)
        return
    if args.only == "qkrope":
        print(json.dumps(run_qkrope(args, dev)), flush=True)
        return
    if args.only == "metadata":
        print(json.dumps(run_metadata(args, dev)), flush=True)
        return
    print(f"[bench] decode workload: bs 64, Hq 32, Hk 8, ctx U[2048,8192], pool 4096 blocks",
          file=sys.stderr, flush=True)
    wl, sets, r = run_decode(args, dev)
    print(f"[bench] decode done: {r['decode_ms'] * 1e3:.1f} us/decode, "
          f"split {r['split_ms'] * 1e3:.1f} us, parity err {r['parity_max_abs_err']:.3e}",
          file=sys.stderr, flush=True)
    fp8 = run_decode_fp8(args, dev, wl, sets)
    print(f"[bench] fp8 decode done: {fp8['decode_fp8_us']} us/decode "
          f"({fp8['decode_fp8_gbs']} GB/s)", file=sys.stderr, flush=True)
    if args.only == "decode":
        print(json.dumps({**r, **fp8}), flush=True)
        return
    comp = run_compress(args, dev)
    print(f"[bench] compress done: {comp['compress_step_us']} us", file=sys.stderr, flush=True)
    pre = run_prefill(args, dev)
    print(f"[bench] prefill done: {pre['prefill_tflops']} / {pre['prefill_chunked_tflops']} "
          f"TFLOP/s", file=sys.stderr, flush=True)
    longctx = run_longctx(args, dev)
    print(f"[bench] long-context decode done: {longctx['longctx_decode_gbs']} GB/s",
          file=sys.stderr, flush=True)
    qkrope = run_qkrope(args, dev)
    print(f"[bench] norm+rope+store done: {qkrope['qkrope_prefill_gbs']} GB/s",
          file=sys.stderr, flush=True)
    meta = run_metadata(args, dev)
    print(f"[bench] metadata done: prefill {meta['metadata_prefill_device_us']} us "
          f"(loop {meta['metadata_prefill_cpu_loop_us']} us)", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(wl, sets[0][0], wl["k_cache"], wl["v_cache"])
        print(f"[bench] cpu baseline done: {cpu['value']} GB/s", file=sys.stderr, flush=True)
    gbs = r["decode_bytes"] / (r["decode_ms"] * 1e-3) / 1e9
    split_gbs = r["split_bytes"] / (r["split_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "store_kvcache (1 token/seq) + paged decode attention, Qwen3-8B "
                        "geometry: Hq 32, Hk 8, head_dim 128, bf16, block 256, batch 64, "
                        "ctx U[2048,8192] (seed 2), pool 4096 blocks, 3 rotated block tables",
            "batch": 64, "n_q_heads": 32, "n_kv_heads": 8, "head_dim": 128, "block_size": 256,
            "parallelism": "single GPU",
        },
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 1),
        "decode_us": round(r["decode_ms"] * 1e3, 2),
        "store_us": round(r["store_ms"] * 1e3, 2),
        "parity_max_abs_err": r["parity_max_abs_err"],
        "roofline": {
            "kernel": DECODE_KERNEL,
            "bound": "hbm",
            "achieved": round(split_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(split_gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(DECODE_PROFILE, DECODE_KERNEL),
            "avg_us": round(r["split_ms"] * 1e3, 2),
            "algorithmic_bytes": r["split_bytes"],
        },
        "cpu_baseline": cpu,
        **comp,
        "prefill_roofline": {
            "kernel": "prefill_varlen_kernel<false, 128, false, true>",
            "bound": "mfma",
            "achieved": pre["prefill_chunked_tflops"],
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(pre["prefill_chunked_tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
            "workload": "2048-token chunks after paged prefixes U[0,8192], 16 sequences",
        },
        **pre,
        **longctx,
        **qkrope,
        **meta,
        **fp8,
        "decode_fp8_speedup": round(r["decode_ms"] * 1e3 / fp8["decode_fp8_us"], 2),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
