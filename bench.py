#!/usr/bin/env python3
"""Decode-attention benchmark at BASELINE cfg2 on one MI355X.

Workload: 1 sequence, 32 query heads / 8 KV heads
(GQA 4), head_dim 128, 65536-token context, page size 64, page table a seeded
random permutation of the 1024-page pool, INT8 K/V with per-(token, kv_head)
fp32 scales, fp16-exact Q, 32 splits (2048 tokens each), fp32 partials, LSE
merge, fp16 output.  A step is one decode-attention call through the C ABI:
kvb_decode_attention_fused (one launch: the int8-MFMA split kernel, whose
last work-group per kv head merges and normalizes).  The two-launch
kvb_decode_attention (split kernel + merge kernel) is timed beside it.

Inputs are resident in HBM before timing.  The KV cache of one call is
132 MiB, which fits the 256 MB MALL, so the timed loop rotates over --copies
independent caches (default 4, 553 MB) and every call streams from HBM.

Prints ONE JSON line: value = effective KV GB/s (KV bytes per call / time per
call), ms_per_step = time per call, plus the roofline of the dominant kernel
(the split kernel, timed alone with HIP events on its launch stream) and the
CPU baseline (the reference's FP64 oracle built from its sources, timed on
this host).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

METRIC = "µs/decode-attention call + effective KV HBM GB/s (% of peak) at 64K ctx"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=4)
    ap.add_argument("--split-tokens", type=int, default=2048)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the hipGraph replay (profiling runs)")
    ap.add_argument("--no-five-layer", action="store_true", help="skip the five-layer graph step (configs[4])")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched configs[2] / configs[3] timings")
    ap.add_argument("--no-mma-geometry", action="store_true",
                    help="skip the rows-8 / group-6 / dim-256 / page-32 launch_attention_mma timing")
    ap.add_argument("--no-append", action="store_true", help="skip the paged INT8 append timings")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run known-size copy and read kernels (for scaling rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    import kvbridge_amd as kvb
    from kvbridge_amd import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kvb.load()
    rows, qh, kvh, D, P, T = 1, 32, 8, 128, 64, 65536
    st = args.split_tokens
    caches = []
    for c in range(args.copies):
        shape, t = W.torch_cache(rows, qh, kvh, D, P, T, seed=0x4B56422 + c, device="cuda:0")
        caches.append(t)
    s = shape
    splits = kvb.split_count(s, st)
    rh = s.rows * s.q_heads
    kv_bytes = T * kvh * (2 * D + 8)
    log(f"cfg2: shape={s.as_tuple()} splits={splits} kv_bytes/call={kv_bytes} copies={args.copies}")

    inps = [kvb.device_input(t["q"], t["qpos"], t["kpos"], t["table"], t["k"], t["v"], t["ks"], t["vs"])
            for t in caches]
    scratch = torch.empty(kvb.scratch_elements(s, st), dtype=torch.float32, device=dev)
    m = torch.empty(rh, dtype=torch.float32, device=dev)
    l = torch.empty(rh, dtype=torch.float32, device=dev)
    n = torch.empty(rh * D, dtype=torch.float32, device=dev)
    out = torch.empty(rh * D, dtype=torch.float16, device=dev)
    assert kvb.selected_kernel(s, inps[0], st) == kvb.KVB_KERNEL_TILED_MFMA
    split_kernel = kvb.selected_kernel_name(s, inps[0], st)                  # split-only launch
    fused_kernel = kvb.selected_kernel_name(s, inps[0], st, fused=True)      # the benchmarked call
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    counters = torch.zeros(kvh, dtype=torch.int32, device=dev)  # zeroed once; every call leaves them zero

    def call(i):  # one decode-attention call: single launch, last work-group merges
        kvb.decode_attention_fused(s, inps[i % len(inps)], st, scratch, counters, m, l, n, out, kvb.KVB_OUT_F16,
                                   sp)

    def call_two_launch(i):  # split kernel + merge kernel
        kvb.decode_attention(s, inps[i % len(inps)], st, scratch, m, l, n, out, kvb.KVB_OUT_F16, sp)

    # ---- parity of the benchmarked configuration against the FP64 oracle.
    parity = None
    if not args.no_parity:
        from oracle import oracle as O

        call(0)
        torch.cuda.synchronize()
        t = caches[0]
        host = W.Case(s, t["q"].cpu().numpy(), t["qpos"].cpu().numpy(), t["kpos"].cpu().numpy(),
                      t["table"].cpu().numpy().view(np.uint32), t["k"].cpu().numpy(), t["v"].cpu().numpy(),
                      t["ks"].cpu().numpy(), t["vs"].cpu().numpy())
        ref, vis = O.fp64(host, threads=min(16, os.cpu_count() or 1))
        g = O.gates(out.float().cpu().numpy().reshape(rh, D), ref)
        parity = {"oracle": "fp64", "max_abs": g["max_abs"], "rel_l2": g["rel_l2"], "pass": g["pass"],
                  "strict_3e-6+5e-5": g["strict_pass"]}
        log(f"parity vs FP64 oracle: {parity}")
        if not g["pass"]:
            print(json.dumps({"metric": METRIC, "error": "parity failed", "parity": parity}))
            sys.exit(1)

    # ---- warmup
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()

    # ---- eager loop: K back-to-back calls on one stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        call(i)
    e1.record(stream)
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / args.steps
    e0.record(stream)
    for i in range(args.steps):
        call_two_launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    two_launch_ms = e0.elapsed_time(e1) / args.steps

    # ---- the reference's own entry point on the same workload: launch_attention
    # with its fixed 256-token splits (256 partials per row-head) + merge, as
    # a drop-in caller gets it.
    ref_scratch = torch.empty(kvb.scratch_elements(s), dtype=torch.float32, device=dev)
    for i in range(5):
        kvb.launch_attention(s, inps[i % len(inps)], ref_scratch, m, l, n, sp)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        kvb.launch_attention(s, inps[i % len(inps)], ref_scratch, m, l, n, sp)
    e1.record(stream)
    torch.cuda.synchronize()
    ref_api_ms = e0.elapsed_time(e1) / args.steps
    del ref_scratch

    # ---- hipGraph replay: one graph holds one call per KV copy
    graph_ms = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        gs = torch.cuda.Stream()
        gs.wait_stream(stream)
        with torch.cuda.stream(gs):
            call(0)  # warm the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=gs):
            for c in range(len(inps)):
                kvb.decode_attention_fused(s, inps[c], st, scratch, counters, m, l, n, out, kvb.KVB_OUT_F16,
                                           gs.cuda_stream)
        torch.cuda.synchronize()
        reps = max(1, args.steps // len(inps))
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        graph_ms = e0.elapsed_time(e1) / (reps * len(inps))

    # ---- split kernel alone (dominant kernel): HIP events on its launch
    # stream around back-to-back launches (the average agrees with the
    # rocprofv3 kernel-trace average; events around single launches add
    # several µs of event overhead each).
    def split_only(i):
        kvb.split_attention(s, inps[i % len(inps)], st, scratch, sp)

    for i in range(args.warmup):
        split_only(i)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        split_only(i)
    e1.record(stream)
    torch.cuda.synchronize()
    split_ms = e0.elapsed_time(e1) / args.steps

    # ---- merge kernel alone
    e0.record(stream)
    for i in range(args.steps):
        kvb.merge_finalize(s, scratch, splits, m, l, n, out, kvb.KVB_OUT_F16, sp)
    e1.record(stream)
    torch.cuda.synchronize()
    merge_ms = e0.elapsed_time(e1) / args.steps

    # The headline call time is the better of back-to-back eager calls and
    # hipGraph replay (a decode loop can issue either way); both are reported.
    call_ms = min(eager_ms, graph_ms) if graph_ms is not None else eager_ms
    value = kv_bytes / (call_ms * 1e-3) / 1e9
    split_gbs = kv_bytes / (split_ms * 1e-3) / 1e9
    # Roofline of the dominant (and only) kernel of the call: the fused split
    # kernel; its launch duration is the eager per-call time (HIP events over
    # back-to-back launches on its stream).
    fused_gbs = kv_bytes / (eager_ms * 1e-3) / 1e9
    log(f"two-launch eager {two_launch_ms*1e3:.2f} us/call; launch_attention (256-token splits) "
        f"{ref_api_ms*1e3:.2f} us/call")
    log(f"eager {eager_ms*1e3:.2f} us/call, graph {graph_ms*1e3 if graph_ms else float('nan'):.2f} us/call, "
        f"{split_kernel} {split_ms*1e3:.2f} us/launch ({split_gbs:.0f} GB/s), merge-only {merge_ms*1e3:.2f} us")

    # ---- same-size streaming read: one launch reading the call's KV byte
    # count with nothing else to do (rotated over as many buffers), the
    # practical ceiling of any single launch that streams these bytes.
    sink = torch.zeros(8192, dtype=torch.int32, device=dev)
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count  # one work-group per CU
    probe_bufs = [torch.ones(kv_bytes, dtype=torch.uint8, device=dev) for _ in range(args.copies)]

    def probe(i):
        kvb.hbm_read_probe(probe_bufs[i % len(probe_bufs)], kv_bytes, sink, n_cu, sp)

    for i in range(args.warmup):
        probe(i)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        probe(i)
    e1.record(stream)
    torch.cuda.synchronize()
    probe_us = e0.elapsed_time(e1) * 1e3 / args.steps
    probe_gbs = kv_bytes / (probe_us * 1e-6) / 1e9
    del probe_bufs
    log(f"stream probe: {kv_bytes} B in {probe_us:.2f} us per launch ({probe_gbs:.0f} GB/s)")

    # ---- paged INT8 append (kvb_append_kv), measured before the GB-sized
    # batched caches come and go (after them the same append has measured up
    # to 7x slower in this process): a 4096-token prefill chunk (tokens
    # fill the slots of randomly chosen pages in order, as a paged prefill does)
    # and a one-token decode step into a cfg2-sized pool, fp16 sources.  Bytes
    # moved per token and kv head: 2 x dim fp16 read, 2 x dim int8 + 8 B scales
    # written.
    append = None
    if not args.no_append:
        append = {}
        apages = 1024
        ak = torch.empty((apages, kvh, P, D), dtype=torch.int8, device=dev)
        av = torch.empty((apages, kvh, D, P), dtype=torch.int8, device=dev)
        aks = torch.empty((apages, kvh, P), dtype=torch.float32, device=dev)
        avs = torch.empty((apages, kvh, P), dtype=torch.float32, device=dev)
        for ntok in (4096, 1):
            kn = torch.randn((ntok, kvh, D), device=dev).half()
            vn = torch.randn((ntok, kvh, D), device=dev).half()
            tok = torch.arange(ntok, device=dev)
            slots = (torch.randperm(apages, device=dev)[tok // P] * P + tok % P).to(torch.int32)
            ash = kvb.append_shape(ntok, kvh, D, P, apages, kvb.KVB_SRC_F16)

            def acall():
                kvb.append_kv(ash, kn, vn, slots, ak, av, aks, avs, stream=sp)

            for _ in range(10):
                acall()
            torch.cuda.synchronize()
            areps = max(100, args.steps // 4)
            e0.record(stream)
            for _ in range(areps):
                acall()
            e1.record(stream)
            torch.cuda.synchronize()
            aus = e0.elapsed_time(e1) * 1e3 / areps
            abytes = ntok * kvh * (2 * D * 2 + 2 * D + 8)
            agbs = abytes / (aus * 1e-6) / 1e9
            append[f"{ntok}_tokens"] = {"bytes_per_call": abytes, "us_per_call": round(aus, 3),
                                        "GB/s": round(agbs, 1), "pct_of_peak": round(100.0 * agbs / HBM_PEAK_GBS, 2)}
            log(f"append {ntok} tokens x {kvh} kv heads (fp16 source): {aus:.2f} us ({agbs:.0f} GB/s)")
        del ak, av, aks, avs

    # ---- five independent cfg2 layers, each one fused
    # decode call, captured as one hipGraph step and replayed.
    five = None
    if not args.no_five_layer and not args.no_graph:
        layers = list(range(min(5, len(caches))))
        extra = []
        while len(layers) + len(extra) < 5:
            _, t_ = W.torch_cache(rows, qh, kvh, D, P, T, seed=0x4B56430 + len(extra), device="cuda:0")
            extra.append(t_)
        linps = [inps[i] for i in layers] + [kvb.device_input(t_["q"], t_["qpos"], t_["kpos"], t_["table"], t_["k"],
                                                             t_["v"], t_["ks"], t_["vs"]) for t_ in extra]
        lbufs = [dict(sc=torch.empty_like(scratch), cnt=torch.zeros(kvh, dtype=torch.int32, device=dev),
                      m=torch.empty_like(m), l=torch.empty_like(l), n=torch.empty_like(n),
                      o=torch.empty_like(out)) for _ in linps]
        gs5 = torch.cuda.Stream()
        gs5.wait_stream(stream)

        def five_step(strm):
            for li, b in zip(linps, lbufs):
                kvb.decode_attention_fused(s, li, st, b["sc"], b["cnt"], b["m"], b["l"], b["n"], b["o"],
                                           kvb.KVB_OUT_F16, strm)

        with torch.cuda.stream(gs5):
            five_step(gs5.cuda_stream)
        torch.cuda.synchronize()
        g5 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g5, stream=gs5):
            five_step(gs5.cuda_stream)
        for _ in range(5):
            g5.replay()
        torch.cuda.synchronize()
        reps5 = max(10, args.steps // 5)
        e0.record(stream)
        for _ in range(reps5):
            g5.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        step_us = e0.elapsed_time(e1) * 1e3 / reps5
        five = {"layers": 5, "us_per_step": round(step_us, 3),
                "GB/s": round(5 * kv_bytes / (step_us * 1e-6) / 1e9, 1),
                "pct_of_peak": round(100.0 * 5 * kv_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                "kv_bytes_per_step": 5 * kv_bytes, "graph": True}
        log(f"five-layer graph step: {step_us:.2f} us ({five['GB/s']:.0f} GB/s)")
        del extra, lbufs

    # ---- BASELINE configs[2] (16 ragged sequences) and configs[3] (4 x 131072
    # tokens, GQA 8): the batched call with counters given (one launch where the
    # library chooses it, else split + merge), back to back.  Each cache (about
    # 0.57 GB and 1.1 GB) is larger than the MALL on its own.
    batched = None
    if not args.no_batched:
        batched = {}
        cfgs = (("cfg3", W.CFG3, W.cfg3_lengths(), 0x4B56423), ("cfg4", W.CFG4, W.CFG4["lengths"], 0x4B56424))
        for label, cfg, lengths, seed in cfgs:
            bshape, bt, blens = W.torch_batch(cfg["rows"], cfg["q_heads"], cfg["kv_heads"], cfg["dim"],
                                              cfg["page_tokens"], lengths, seed=seed,
                                              split_tokens=cfg["split_tokens"],
                                              outlier_frac=cfg.get("outlier_frac", 0.0))
            binp = kvb.batch_input(bt["q"], bt["qpos"], bt["starts"], bt["offsets"], bt["kpos"], bt["table"],
                                   bt["k"], bt["v"], bt["ks"], bt["vs"])
            brh = kvb.batch_output_scalar_elements(bshape)
            bsc = torch.empty(kvb.batch_scratch_elements(bshape), dtype=torch.float32, device=dev)
            bcnt = torch.zeros(bshape.batch * bshape.kv_heads, dtype=torch.int32, device=dev)
            bm, bl = torch.empty(brh, dtype=torch.float32, device=dev), torch.empty(brh, dtype=torch.float32,
                                                                                      device=dev)
            bn = torch.empty(brh * bshape.dim, dtype=torch.float32, device=dev)
            bo = torch.empty(brh * bshape.dim, dtype=torch.float16, device=dev)

            def time_mode(counters):
                def bcall():
                    kvb.decode_attention_batched(bshape, binp, bsc, bm, bl, bn, bo, kvb.KVB_OUT_F16,
                                                 counters=counters, stream=sp)

                for _ in range(10):
                    bcall()
                torch.cuda.synchronize()
                breps = max(20, args.steps // 10)
                e0.record(stream)
                for _ in range(breps):
                    bcall()
                e1.record(stream)
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) * 1e3 / breps

            # With counters the library runs one launch where its single-launch
            # kernel serves the shape (else split + merge); without, always
            # split + merge.  Both are timed; the faster is the call's figure.
            bbytes = sum(blens) * bshape.kv_heads * (2 * bshape.dim + 8)
            bkern = kvb.batch_kernel_name(bshape, binp, fused=True)
            launches = 1 if bkern.startswith("split_i8_kernel<") and bkern.split(",")[5] == "true" else 2
            modes = {"with_counters": time_mode(bcnt)}
            if launches == 1:
                modes["split_merge"] = time_mode(None)
            best = min(modes, key=modes.get)
            bus = modes[best]
            bgbs = bbytes / (bus * 1e-6) / 1e9
            batched[label] = {"sequences": bshape.batch, "tokens": sum(blens), "q_heads": bshape.q_heads,
                              "kv_bytes_per_call": bbytes, "us_per_call": round(bus, 3), "GB/s": round(bgbs, 1),
                              "pct_of_peak": round(100.0 * bgbs / HBM_PEAK_GBS, 2),
                              "kernel": bkern if best == "with_counters" else kvb.batch_kernel_name(bshape, binp),
                              "launches": launches if best == "with_counters" else 2,
                              "split_tokens": bshape.split_tokens,
                              "splits_per_seq_max": kvb.batch_split_count(bshape),
                              "us_by_mode": {k: round(v, 3) for k, v in modes.items()}}
            log(f"{label} batched call ({batched[label]['launches']} launch"
                f"{'es' if batched[label]['launches'] > 1 else ''}, {batched[label]['kernel']}, "
                f"{bshape.split_tokens}-token splits): {bus:.2f} us ({bgbs:.0f} GB/s, "
                f"{100.0 * bgbs / HBM_PEAK_GBS:.1f}% of peak); modes {batched[label]['us_by_mode']}")
            del bt, bsc, bm, bl, bn, bo, bcnt
            torch.cuda.empty_cache()

    # ---- the reference's dense MMA geometry (attention_mma_supported: 8 query
    # rows sharing the KV, 24 q / 4 kv heads = group 6, dim 256, page 32) at
    # 65536 tokens: launch_attention_mma (its 256-token splits + merge), back
    # to back over rotated caches.  KV bytes per call 136,314,880, the byte
    # count of the reference's own 64K benchmark (data/att-bench-65536-v2-07.json).
    mma = None
    if not args.no_mma_geometry:
        mcaches = [W.torch_cache(8, 24, 4, 256, 32, 65536, seed=0x4B56440 + c, device="cuda:0")
                   for c in range(args.copies)]
        ms_ = mcaches[0][0]
        assert kvb.attention_mma_supported(ms_)
        minps = [kvb.device_input(t_["q"], t_["qpos"], t_["kpos"], t_["table"], t_["k"], t_["v"], t_["ks"], t_["vs"])
                 for _, t_ in mcaches]
        mrh = ms_.rows * ms_.q_heads
        msc = torch.empty(kvb.scratch_elements(ms_), dtype=torch.float32, device=dev)
        mm_, ml_ = torch.empty(mrh, device=dev), torch.empty(mrh, device=dev)
        mn_ = torch.empty(mrh * ms_.dim, device=dev)

        def mcall(i):
            kvb.launch_attention_mma(ms_, minps[i % len(minps)], msc, mm_, ml_, mn_, sp)

        for i in range(10):
            mcall(i)
        torch.cuda.synchronize()
        mreps = max(50, args.steps // 4)
        e0.record(stream)
        for i in range(mreps):
            mcall(i)
        e1.record(stream)
        torch.cuda.synchronize()
        mus = e0.elapsed_time(e1) * 1e3 / mreps
        mbytes = 65536 * ms_.kv_heads * (2 * ms_.dim + 8)
        mgbs = mbytes / (mus * 1e-6) / 1e9
        mma = {"shape": "8 rows x 24 q / 4 kv heads, dim 256, page 32, 65536 tokens, 256 splits + merge",
               "kv_bytes_per_call": mbytes, "us_per_call": round(mus, 3), "GB/s": round(mgbs, 1),
               "pct_of_peak": round(100.0 * mgbs / HBM_PEAK_GBS, 2),
               "kernel": kvb.selected_kernel_name(ms_, minps[0], 256)}
        log(f"mma geometry (launch_attention_mma): {mus:.2f} us ({mgbs:.0f} GB/s, "
            f"{100.0 * mgbs / HBM_PEAK_GBS:.1f}% of peak)")
        # The same geometry through kvb_decode_attention with 1024-token
        # splits: one work-group per (split, kv head) for every CU, a quarter
        # of the partials to write and merge.
        dst_ = 1024

        def dcall(i):
            kvb.decode_attention(ms_, minps[i % len(minps)], dst_, msc, mm_, ml_, mn_, stream=sp)

        for i in range(10):
            dcall(i)
        torch.cuda.synchronize()
        e0.record(stream)
        for i in range(mreps):
            dcall(i)
        e1.record(stream)
        torch.cuda.synchronize()
        dus = e0.elapsed_time(e1) * 1e3 / mreps
        dgbs = mbytes / (dus * 1e-6) / 1e9
        mma["decode_1024_token_splits"] = {
            "splits": kvb.split_count(ms_, dst_), "us_per_call": round(dus, 3), "GB/s": round(dgbs, 1),
            "pct_of_peak": round(100.0 * dgbs / HBM_PEAK_GBS, 2), "kernel": kvb.selected_kernel_name(ms_, minps[0], dst_)}
        log(f"mma geometry (decode_attention, {dst_}-token splits): {dus:.2f} us ({dgbs:.0f} GB/s, "
            f"{100.0 * dgbs / HBM_PEAK_GBS:.1f}% of peak)")
        del mcaches, minps, msc
        torch.cuda.empty_cache()

    # ---- known-size kernels for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE
    if args.calibrate:
        cal_bytes = 256 << 20
        src = torch.empty(cal_bytes, dtype=torch.uint8, device=dev)
        dst = torch.empty(cal_bytes, dtype=torch.uint8, device=dev)
        sink = torch.zeros(8192, dtype=torch.int32, device=dev)
        for _ in range(5):
            dst.copy_(src)                                   # reads and writes cal_bytes
            kvb.hbm_read_probe(src, cal_bytes, sink, n_cu)   # reads cal_bytes
        torch.cuda.synchronize()
        log(f"calibration: 5 x copy of {cal_bytes} B and 5 x read probe of {cal_bytes} B")

    # ---- HBM traffic per split launch, from committed rocprofv3 counter runs
    traffic = None
    tpath = os.path.join(root, "profiles", "traffic_cfg2.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            tinfo = json.load(fh)
        if tinfo.get("kernel") == fused_kernel:
            traffic = tinfo.get("hbm_bytes_per_launch")

    # ---- CPU baseline: the reference's FP64 oracle on this host
    cpu = None
    if not args.no_cpu_baseline and not args.no_parity:
        from oracle import oracle as O

        kind = "reference" if O.ref_available() else "port"
        fn = O.ref_fp64 if kind == "reference" else (lambda c: O.fp64(c, threads=1))
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 50):
            t0 = time.perf_counter()
            fn(host)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        cpu = {"value": kv_bytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
               "us_per_call": med * 1e6,
               "sample": f"{len(times)} full cfg2 calls (FP64 scalar oracle, examples/attention_reference.h), median"}
        log(f"cpu baseline ({kind}): {med*1e3:.1f} ms/call")

    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(call_ms, 6),
        "us_per_call": round(call_ms * 1e3, 3),
        "pct_of_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "eager_us_per_call": round(eager_ms * 1e3, 3),
        "two_launch_eager_us_per_call": round(two_launch_ms * 1e3, 3),
        "launch_attention_256_token_splits_us_per_call": round(ref_api_ms * 1e3, 3),
        "graph_us_per_call": round(graph_ms * 1e3, 3) if graph_ms is not None else None,
        "merge_kernel_us": round(merge_ms * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic",
        "config": {"workload": "cfg2: 1 seq, 32q/8kv heads, d128, 65536 tokens, page 64, random 1024-page "
                               "permutation, int8 KV + per-(token,kv_head) fp32 scales, 32 splits, fp16 out",
                   "kv_copies_rotated": args.copies, "kv_bytes_per_call": kv_bytes, "split_tokens": st,
                   "splits": splits},
        "roofline": {"bound": "hbm", "achieved": round(fused_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(fused_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": fused_kernel, "algorithmic_bytes_per_launch": kv_bytes,
                     "launch_us": round(eager_ms * 1e3, 3)},
        "split_only": {"kernel": split_kernel, "us": round(split_ms * 1e3, 3), "GB/s": round(split_gbs, 1)},
        "stream_probe": {"bytes": kv_bytes, "us": round(probe_us, 3), "GB/s": round(probe_gbs, 1),
                         "pct_of_peak": round(100.0 * probe_gbs / HBM_PEAK_GBS, 2),
                         "note": "one plain streaming-read launch of the call's KV byte count, rotated buffers"},
        "five_layer_step": five,
        "batched": batched,
        "mma_geometry": mma,
        "append": append,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
