#!/usr/bin/env python3
"""Decode-attention benchmark at BASELINE cfg2 on one MI355X.

Workload: 1 sequence, 32 query heads / 8 KV heads
(GQA 4), head_dim 128, 65536-token context, page size 64, page table a seeded
random permutation of the 1024-page pool, INT8 K/V with per-(token, kv_head)
fp32 scales, fp16-exact Q, 32 splits (2048 tokens each), fp32 partials, LSE
merge, fp16 output.  A step is one decode-attention call through the C ABI:
kvb_decode_attention_fused (one launch: the int8-MFMA split kernel, whose
last work-group per kv head merges and normalizes).

Inputs are resident in HBM before timing.  The KV cache of one call is
132 MiB, which fits the 256 MB MALL, so every timed loop rotates over --copies
independent caches (default 8, 1.1 GB) and every call streams from HBM.

Method, per timed section:
  * gate first: the section's output is checked against the FP64 oracle
    (append: bitwise against the CPU quantizer) before anything is timed; a
    failing gate prints an error line and exits 1 (reference
    examples/attention_bench.cu:133-149, :197-199);
  * settle: --settle-seconds of back-to-back calls bring the GPU to its
    steady clock and warm the address translation of every copy (a 20-call
    loop right after an idle host phase otherwise measures the ramp);
  * --warmup calls, then exactly --steps calls timed back to back with HIP
    events on the launch stream;
  * repeat check: after timing, each copy's output must be bitwise equal to
    its output before timing (attention_bench.cu:224-226);
  * the headline call also gets the reference's per-iteration statistics:
    8 warmup calls, then 32 calls each bracketed by its own events and a
    sync, p50 / p95 (attention_bench.cu:187-231, bench_options.h:8).

Prints ONE JSON line: value = effective KV GB/s (KV bytes per call / time per
call), ms_per_step = time per call (back-to-back eager calls), the roofline of
the call's only kernel, and the CPU baselines (the reference's FP64 oracle
built from its sources, 1 core; a threaded fp32 split-K + merge restatement
on the host's cores) timed on this host.
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


def fail(msg, **extra):
    print(json.dumps({"metric": METRIC, "error": msg, **extra}), flush=True)
    sys.exit(1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--split-tokens", type=int, default=2048)
    ap.add_argument("--settle-seconds", type=float, default=0.25,
                    help="back-to-back calls before each timed section (GPU clock, address translation)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the FP64 CPU baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=0, help="threads of the fp32 CPU baseline (0: all)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-parity", action="store_true", help="skip the gates (profiling runs only)")
    ap.add_argument("--no-graph", action="store_true", help="skip the hipGraph replays (profiling runs)")
    ap.add_argument("--no-fenced", action="store_true",
                    help="skip the fenced-ticket diagnostic single launch (kvb_decode_attention_fused_fenced)")
    ap.add_argument("--no-five-layer", action="store_true", help="skip the five-layer graph step (configs[4])")
    ap.add_argument("--five-layer-only", action="store_true",
                    help="run only the five-layer graph step and its eager comparison (kernel-trace runs)")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched configs[2] / configs[3] timings")
    ap.add_argument("--no-mma-geometry", action="store_true",
                    help="skip the rows-8 / group-6 / dim-256 / page-32 launch_attention_mma timing")
    ap.add_argument("--mma-calls", choices=("both", "launch_attention_mma", "decode_1024_token_splits"),
                    default="both", help="which dense-geometry calls to time (profiling runs select one)")
    ap.add_argument("--no-append", action="store_true", help="skip the paged INT8 append timings")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run known-size copy and read kernels (for scaling rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)

    # hipGraph launch path of the HIP runtime: its default pre-recorded
    # packet submission adds about 0.8 us between consecutive kernel nodes of
    # this length (measured: five-layer step 137.8 us against 134.8 us with it
    # off, eager 133.6 us); set before the runtime initializes, overridable.
    os.environ.setdefault("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "0")
    import numpy as np
    import torch

    root = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, root)
    import kvbridge_amd as kvb
    from kvbridge_amd import workloads as W

    gate = not args.no_parity
    if gate:
        from oracle import oracle as O
    host_threads = min(16, len(os.sched_getaffinity(0)))

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kvb.load()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, steps):
        """ms per call of `steps` back-to-back calls fn(i), HIP events on the
        launch stream.  One untimed call fn(-1) is queued before the start
        event, so the span opens when the device is already busy and holds
        exactly `steps` calls of device time: the host's first submission
        (up to tens of us for a graph launch) is not inside it."""
        torch.cuda.synchronize()
        fn(-1)
        e0.record(stream)
        for i in range(steps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def settle(fn, seconds=None):
        """Untimed back-to-back calls for `seconds` (GPU clock, translation of every copy)."""
        seconds = args.settle_seconds if seconds is None else seconds
        torch.cuda.synchronize()
        t0, i = time.perf_counter(), 0
        while True:
            for _ in range(32):
                fn(i)
                i += 1
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= seconds:
                return i

    def warm_and_time(fn, steps=None, warmup=None):
        settle(fn)
        for i in range(args.warmup if warmup is None else warmup):
            fn(i)
        return timed(fn, args.steps if steps is None else steps)

    def bits(t):
        return t.detach().cpu().numpy().view(np.uint8).copy()

    def gbs(nbytes, us):
        return nbytes / (us * 1e-6) / 1e9

    # ------------------------------------------------------------------ cfg2
    rows, qh, kvh, D, P, T = 1, 32, 8, 128, 64, 65536
    st = args.split_tokens
    copies = max(1, args.copies)
    caches = []
    for c in range(copies):
        shape, t = W.torch_cache(rows, qh, kvh, D, P, T, seed=0x4B56422 + c, device="cuda:0")
        caches.append(t)
    s = shape
    splits = kvb.split_count(s, st)
    rh = s.rows * s.q_heads
    kv_bytes = T * kvh * (2 * D + 8)
    log(f"cfg2: shape={s.as_tuple()} splits={splits} kv_bytes/call={kv_bytes} copies={copies}")

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
    counters = torch.zeros(kvh, dtype=torch.int32, device=dev)  # zeroed once; every call leaves them zero

    def call(i):  # one decode-attention call: single launch, last work-group merges
        kvb.decode_attention_fused(s, inps[i % copies], st, scratch, counters, m, l, n, out, kvb.KVB_OUT_F16, sp)

    def call_two_launch(i):  # split kernel + merge kernel
        kvb.decode_attention(s, inps[i % copies], st, scratch, m, l, n, out, kvb.KVB_OUT_F16, sp)

    def outputs_of(fn):
        """Each copy's output bits after one call of fn on it."""
        res = []
        for c in range(copies):
            fn(c)
            torch.cuda.synchronize()
            res.append(bits(out))
        return res

    def same(a, b):
        return all(np.array_equal(x, y) for x, y in zip(a, b))

    host_case = {}

    def fp64_ref(c):
        if c not in host_case:
            t = caches[c]
            case = W.Case(s, t["q"].cpu().numpy(), t["qpos"].cpu().numpy(), t["kpos"].cpu().numpy(),
                          t["table"].cpu().numpy().view(np.uint32), t["k"].cpu().numpy(), t["v"].cpu().numpy(),
                          t["ks"].cpu().numpy(), t["vs"].cpu().numpy())
            host_case[c] = (case, O.fp64(case, threads=host_threads))
        return host_case[c]

    def gate_out(label, out_f32, c=0, bits0=None):
        """North-star gate of a normalized [rh, D] output against FP64 (copy
        c); bits0: the fp16 output's bytes instead of out_f32."""
        if bits0 is not None:
            out_f32 = bits0.view(np.float16).astype(np.float32)
        _, (ref, _) = fp64_ref(c)
        g = O.gates(out_f32.reshape(-1, D), ref)
        res = {"oracle": "fp64", "max_abs": g["max_abs"], "rel_l2": g["rel_l2"], "pass": bool(g["pass"]),
               "strict_3e-6+5e-5": bool(g["strict_pass"])}
        log(f"gate {label}: {res}")
        if not g["pass"]:
            fail(f"parity failed: {label}", parity=res)
        return res

    def five_layer_step():
        """five independent cfg2 layers (copies 0..4),
        each one fused decode call, captured as one hipGraph step and
        replayed; every layer gated, replays bitwise equal to the eager step."""
        five = {}
        layers = list(range(min(5, copies)))
        extra = []
        while len(layers) + len(extra) < 5:
            _, t_ = W.torch_cache(rows, qh, kvh, D, P, T, seed=0x4B56430 + len(extra), device="cuda:0")
            extra.append(t_)
        linps = [inps[i] for i in layers] + [kvb.device_input(t_["q"], t_["qpos"], t_["kpos"], t_["table"], t_["k"],
                                                             t_["v"], t_["ks"], t_["vs"]) for t_ in extra]
        lbufs = [dict(sc=torch.empty_like(scratch), cnt=torch.zeros(kvh, dtype=torch.int32, device=dev),
                      m=torch.empty_like(m), l=torch.empty_like(l), n=torch.empty_like(n),
                      o=torch.empty_like(out)) for _ in linps]

        def five_step(strm):
            for li, b in zip(linps, lbufs):
                kvb.decode_attention_fused(s, li, st, b["sc"], b["cnt"], b["m"], b["l"], b["n"], b["o"],
                                           kvb.KVB_OUT_F16, strm)

        five_step(sp)
        torch.cuda.synchronize()
        eager_layers = [bits(b["o"]) for b in lbufs]
        if gate:
            five["parity"] = [gate_out(f"five-layer step, layer {k} (eager)", lbufs[k]["o"].float().cpu().numpy(),
                                       c=layers[k])
                              for k in range(len(layers))]
        gs5 = torch.cuda.Stream()
        gs5.wait_stream(stream)
        with torch.cuda.stream(gs5):
            five_step(gs5.cuda_stream)
        torch.cuda.synchronize()
        g5 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g5, stream=gs5):
            five_step(gs5.cuda_stream)
        step_ms = warm_and_time(lambda i: g5.replay(), steps=max(64, args.steps // 5), warmup=5)
        replay_ok = all(np.array_equal(bits(b["o"]), e) for b, e in zip(lbufs, eager_layers))
        if not replay_ok:
            fail("five-layer graph replay differs from the eager step")
        eager_step_ms = warm_and_time(lambda i: five_step(sp), steps=max(64, args.steps // 5), warmup=5)
        # The same step captured twice into one graph: what one replay costs
        # beyond its kernels (the step graph against two steps per replay).
        g10 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g10, stream=gs5):
            five_step(gs5.cuda_stream)
            five_step(gs5.cuda_stream)
        two_step_ms = warm_and_time(lambda i: g10.replay(), steps=max(32, args.steps // 10), warmup=3) / 2
        if not all(np.array_equal(bits(b["o"]), e) for b, e in zip(lbufs, eager_layers)):
            fail("two-step graph replay differs from the eager step")
        step_us = step_ms * 1e3
        five.update({"layers": 5, "us_per_step": round(step_us, 3), "GB/s": round(gbs(5 * kv_bytes, step_us), 1),
                     "pct_of_peak": round(100.0 * gbs(5 * kv_bytes, step_us) / HBM_PEAK_GBS, 2),
                     "kv_bytes_per_step": 5 * kv_bytes, "graph": True, "replay_bitwise_equal_to_eager": replay_ok,
                     "eager_us_per_step": round(eager_step_ms * 1e3, 3),
                     "two_steps_per_replay_us_per_step": round(two_step_ms * 1e3, 3),
                     "replay_overhead_us": round(2e3 * (step_ms - two_step_ms), 3)})
        log(f"five-layer graph step: {step_us:.2f} us ({five['GB/s']:.0f} GB/s); eager {eager_step_ms*1e3:.2f} us; "
            f"two steps per replay {two_step_ms*1e3:.2f} us per step")
        del extra, lbufs, g5, g10
        return five

    if args.five_layer_only:  # profiling runs: this leg alone, one JSON line
        print(json.dumps({"metric": METRIC, "five_layer_step": five_layer_step()}), flush=True)
        return

    # ---- gate of the benchmarked call, then the headline timing
    parity = None
    if gate:
        call(0)
        torch.cuda.synchronize()
        parity = gate_out("fused call (copy 0)", out.float().cpu().numpy())
    before = outputs_of(call)
    settle_calls = settle(call)
    for i in range(args.warmup):
        call(i)
    eager_ms = timed(call, args.steps)                                       # the headline: exactly K steps
    repeat_ok = same(before, outputs_of(call))
    if not repeat_ok:
        fail("fused call output changed between calls (repeat check)")
    # per-iteration events (the reference's method): 8 warmup, 32 iterations
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(32)]
    for i in range(8):
        call(i)
    torch.cuda.synchronize()
    per_iter = []
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        call(i)
        b.record(stream)
        b.synchronize()
        per_iter.append(a.elapsed_time(b) * 1e3)
    per_iter.sort()
    p50, p95 = statistics.median(per_iter), per_iter[int(math.ceil(0.95 * len(per_iter))) - 1]
    log(f"fused call: {eager_ms*1e3:.2f} us/call back to back ({args.steps} calls after {settle_calls} settle + "
        f"{args.warmup} warmup); per-iteration events p50 {p50:.2f} p95 {p95:.2f} us; repeat bitwise {repeat_ok}")

    # ---- diagnostic: the same single launch with formal release / acquire
    # fences around the merge ticket (kvb_decode_attention_fused_fenced), the
    # ordering the benchmarked call replaces with agent-scope atomic partials.
    fenced = None
    if not args.no_fenced:
        def call_fenced(i):
            kvb.decode_attention_fused_fenced(s, inps[i % copies], st, scratch, counters, m, l, n, out,
                                              kvb.KVB_OUT_F16, sp)

        fenced = {"kernel": "split_i8_kernel<128,8,2,true,4,true,false,true>"}
        before_f = outputs_of(call_fenced)
        fenced["bitwise_equal_to_fused"] = same(before, before_f)
        if not fenced["bitwise_equal_to_fused"]:
            fail("fenced single launch differs from the benchmarked call")
        if gate:
            fenced["parity"] = gate_out("fenced single launch (copy 0)", None, c=0, bits0=before_f[0])
        fenced["us_per_call"] = round(warm_and_time(call_fenced) * 1e3, 3)
        log(f"fenced single launch (diagnostic): {fenced['us_per_call']:.2f} us/call")

    # ---- two launches: split kernel + merge kernel
    two = {}
    if gate:
        call_two_launch(0)
        torch.cuda.synchronize()
        two["parity"] = gate_out("two-launch call (copy 0)", out.float().cpu().numpy())
    before2 = outputs_of(call_two_launch)
    two_ms = warm_and_time(call_two_launch)
    two["us_per_call"] = round(two_ms * 1e3, 3)
    two["repeat_bitwise"] = same(before2, outputs_of(call_two_launch))
    two["bitwise_equal_to_fused"] = same(before, before2)
    if not two["repeat_bitwise"]:
        fail("two-launch output changed between calls (repeat check)")
    log(f"two-launch call: {two_ms*1e3:.2f} us/call")

    # ---- the reference's own entry point: launch_attention, 256-token splits + merge
    ref_api = {}
    ref_scratch = torch.empty(kvb.scratch_elements(s), dtype=torch.float32, device=dev)

    def ref_call(i):
        kvb.launch_attention(s, inps[i % copies], ref_scratch, m, l, n, sp)

    if gate:
        ref_call(0)
        torch.cuda.synchronize()
        o_, vis_, ok_ = O.normalize(m.cpu().numpy(), l.cpu().numpy(), n.cpu().numpy(), D)
        if not ok_:
            fail("launch_attention: empty-row convention violated")
        ref_api["parity"] = gate_out("launch_attention (copy 0)", o_)
    ref_ms = warm_and_time(ref_call)
    ref_api["us_per_call"] = round(ref_ms * 1e3, 3)
    ref_api["splits"] = kvb.split_count(s)
    log(f"launch_attention (256-token splits): {ref_ms*1e3:.2f} us/call")
    del ref_scratch

    # ---- hipGraph replay: one graph holds one fused call per KV copy
    graph = None
    if not args.no_graph:
        g = torch.cuda.CUDAGraph()
        gs = torch.cuda.Stream()
        gs.wait_stream(stream)
        with torch.cuda.stream(gs):
            call(0)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=gs):
            for c in range(copies):
                kvb.decode_attention_fused(s, inps[c], st, scratch, counters, m, l, n, out, kvb.KVB_OUT_F16,
                                           gs.cuda_stream)
        torch.cuda.synchronize()
        reps = max(64, -(-args.steps // copies))  # at least 64 replays, whatever --steps
        gms = warm_and_time(lambda i: g.replay(), steps=reps, warmup=3) / copies
        graph_ok = np.array_equal(bits(out), before[copies - 1])
        if not graph_ok:
            fail("graph replay output differs from the eager call")
        graph = {"us_per_call": round(gms * 1e3, 3), "calls_per_graph": copies, "replays": reps,
                 "bitwise_equal_to_eager": graph_ok}
        log(f"graph replay: {gms*1e3:.2f} us/call")
        del g

    # ---- split kernel alone (the single launch minus its merge tail) and merge kernel alone
    def split_only(i):
        kvb.split_attention(s, inps[i % copies], st, scratch, sp)

    split_ms = warm_and_time(split_only)

    def merge_only(i):
        kvb.merge_finalize(s, scratch, splits, m, l, n, out, kvb.KVB_OUT_F16, sp)

    merge_ms = warm_and_time(merge_only)
    log(f"{split_kernel}: {split_ms*1e3:.2f} us/launch ({gbs(kv_bytes, split_ms*1e3):.0f} GB/s); "
        f"merge-only {merge_ms*1e3:.2f} us")

    # ---- read probes: the call's byte count streamed contiguously (the
    # practical ceiling of one launch), and the call's own KV bytes read
    # through its page table with the decode work split and no arithmetic
    # (the floor of the paged access pattern).
    sink = torch.zeros(8192, dtype=torch.int32, device=dev)
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    probe_bufs = [torch.ones(kv_bytes, dtype=torch.uint8, device=dev) for _ in range(copies)]
    probe_ms = warm_and_time(lambda i: kvb.hbm_read_probe(probe_bufs[i % copies], kv_bytes, sink, n_cu, sp))
    del probe_bufs
    paged_ms = warm_and_time(lambda i: kvb.paged_read_probe(s, inps[i % copies], st, sink, sp))
    log(f"stream probe: {probe_ms*1e3:.2f} us ({gbs(kv_bytes, probe_ms*1e3):.0f} GB/s); paged probe "
        f"{paged_ms*1e3:.2f} us ({gbs(kv_bytes, paged_ms*1e3):.0f} GB/s)")

    # ---- paged INT8 append (kvb_append_kv): 4096- and 16384-token prefill
    # chunks (tokens fill randomly chosen pages in order, as a paged prefill
    # does) and a one-token decode step into a cfg2-sized pool, fp16 sources.  Gated
    # bitwise against the CPU quantizer; timed as a captured graph of 32
    # appends (device time per append, not Python submission).  Bytes per
    # token and kv head: 2 x dim fp16 read, 2 x dim int8 + 8 B scales written.
    append = None
    if not args.no_append:
        append = {}
        apages = 1024
        ak = torch.zeros((apages, kvh, P, D), dtype=torch.int8, device=dev)
        av = torch.zeros((apages, kvh, D, P), dtype=torch.int8, device=dev)
        aks = torch.zeros((apages, kvh, P), dtype=torch.float32, device=dev)
        avs = torch.zeros((apages, kvh, P), dtype=torch.float32, device=dev)
        gen = torch.Generator(device=dev)
        gen.manual_seed(0x4B56450)
        for ntok in (4096, 16384, 1):
            kn = torch.randn((ntok, kvh, D), generator=gen, device=dev).half()
            vn = torch.randn((ntok, kvh, D), generator=gen, device=dev).half()
            tok = torch.arange(ntok, device=dev)
            slots = (torch.randperm(apages, generator=gen, device=dev)[tok // P] * P + tok % P).to(torch.int32)
            ash = kvb.append_shape(ntok, kvh, D, P, apages, kvb.KVB_SRC_F16)

            def acall(i=0):
                kvb.append_kv(ash, kn, vn, slots, ak, av, aks, avs, stream=sp)

            rec = {}
            if gate:
                for tt in (ak, av, aks, avs):
                    tt.zero_()
                acall()
                torch.cuda.synchronize()
                hk, hv, hks, hvs = O.append_int8(np.zeros(ak.shape, np.int8), np.zeros(av.shape, np.int8),
                                                 np.zeros(aks.shape, np.float32), np.zeros(avs.shape, np.float32),
                                                 kn.float().cpu().numpy(), vn.float().cpu().numpy(),
                                                 slots.cpu().numpy().view(np.uint32), P)
                ok = (np.array_equal(hk, ak.cpu().numpy()) and np.array_equal(hv, av.cpu().numpy()) and
                      np.array_equal(hks.view(np.uint32), aks.cpu().numpy().view(np.uint32)) and
                      np.array_equal(hvs.view(np.uint32), avs.cpu().numpy().view(np.uint32)))
                log(f"gate append {ntok} tokens: bitwise {ok}")
                if not ok:
                    fail(f"append of {ntok} tokens differs from the CPU quantizer")
                rec["parity"] = {"oracle": "cpu quantizer", "bitwise": True}
            eager_us = warm_and_time(acall, steps=max(100, args.steps // 4)) * 1e3
            gus = None
            if not args.no_graph:
                ga = torch.cuda.CUDAGraph()
                gsa = torch.cuda.Stream()
                gsa.wait_stream(stream)
                with torch.cuda.stream(gsa):
                    acall()
                torch.cuda.synchronize()
                per_graph = 32
                with torch.cuda.graph(ga, stream=gsa):
                    for _ in range(per_graph):
                        kvb.append_kv(ash, kn, vn, slots, ak, av, aks, avs, stream=gsa.cuda_stream)
                gus = warm_and_time(lambda i: ga.replay(), steps=max(10, args.steps // 32), warmup=3) * 1e3 / per_graph
                del ga
            abytes = ntok * kvh * (2 * D * 2 + 2 * D + 8)
            aus = gus if gus is not None else eager_us
            rec.update({"bytes_per_call": abytes, "us_per_call": round(aus, 3), "GB/s": round(gbs(abytes, aus), 1),
                        "pct_of_peak": round(100.0 * gbs(abytes, aus) / HBM_PEAK_GBS, 2),
                        "timing": "graph of 32 appends, per append" if gus is not None else "eager",
                        "eager_us_per_call": round(eager_us, 3)})
            append[f"{ntok}_tokens"] = rec
            log(f"append {ntok} tokens x {kvh} kv heads (fp16 source): {aus:.2f} us per append "
                f"({gbs(abytes, aus):.0f} GB/s); eager loop {eager_us:.2f} us")
        del ak, av, aks, avs

    # ---- five independent cfg2 layers in one hipGraph step
    five = None
    if not args.no_five_layer and not args.no_graph:
        five = five_layer_step()

    # ---- BASELINE configs[2] (16 ragged sequences) and configs[3] (4 x 131072
    # tokens, GQA 8): the batched call, with counters given (one launch where
    # the library chooses it, else split + merge) and without.  Each cache
    # (about 0.57 GB and 1.1 GB) is larger than the MALL on its own.
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
            rec = {}

            def bcall_of(cnt):
                def bcall(i=0):
                    kvb.decode_attention_batched(bshape, binp, bsc, bm, bl, bn, bo, kvb.KVB_OUT_F16,
                                                 counters=cnt, stream=sp)
                return bcall

            if gate:
                bcall_of(bcnt)()
                torch.cuda.synchronize()
                host = W.batch_to_host(bshape, bt, blens)
                mh, lh, nh = bm.cpu().numpy(), bl.cpu().numpy(), bn.cpu().numpy().reshape(-1, bshape.dim)
                worst = {"max_abs": 0.0, "rel_l2": 0.0}
                brh1 = bshape.rows * bshape.q_heads
                for b in range(bshape.batch):
                    sl = slice(b * brh1, (b + 1) * brh1)
                    case = host.sequence(b)
                    ref, _ = O.fp64(case, threads=host_threads)
                    o_, _, ok_ = O.normalize(mh[sl], lh[sl], nh[sl].ravel(), bshape.dim)
                    g_ = O.gates(o_, ref)
                    if not ok_ or not g_["pass"]:
                        fail(f"parity failed: {label} sequence {b}", parity=g_)
                    worst["max_abs"] = max(worst["max_abs"], g_["max_abs"])
                    worst["rel_l2"] = max(worst["rel_l2"], g_["rel_l2"])
                rec["parity"] = {"oracle": "fp64", "sequences": bshape.batch, "pass": True, **worst}
                log(f"gate {label}: every sequence passes, worst {worst}")
                del host
            modes = {}
            for mode, cnt in (("with_counters", bcnt), ("split_merge", None)):
                fn = bcall_of(cnt)
                fn()
                torch.cuda.synchronize()
                before_b = bits(bo)
                modes[mode] = warm_and_time(fn, steps=max(20, args.steps // 10), warmup=10) * 1e3
                fn()
                torch.cuda.synchronize()
                if not np.array_equal(before_b, bits(bo)):
                    fail(f"{label} ({mode}) output changed between calls (repeat check)")
            bkern = kvb.batch_kernel_name(bshape, binp, fused=True)
            launches = 1 if bkern.startswith("split_i8_kernel<") and bkern.split(",")[5] == "true" else 2
            best = min(modes, key=modes.get)
            bus = modes[best]
            bbytes = sum(blens) * bshape.kv_heads * (2 * bshape.dim + 8)
            rec.update({"sequences": bshape.batch, "tokens": sum(blens), "q_heads": bshape.q_heads,
                        "kv_bytes_per_call": bbytes, "us_per_call": round(bus, 3), "GB/s": round(gbs(bbytes, bus), 1),
                        "pct_of_peak": round(100.0 * gbs(bbytes, bus) / HBM_PEAK_GBS, 2),
                        "kernel": bkern if best == "with_counters" else kvb.batch_kernel_name(bshape, binp),
                        "launches": launches if best == "with_counters" else 2,
                        "split_tokens": bshape.split_tokens, "splits_per_seq_max": kvb.batch_split_count(bshape),
                        "us_by_mode": {k: round(v, 3) for k, v in modes.items()}, "repeat_bitwise": True})
            batched[label] = rec
            log(f"{label} batched call ({rec['launches']} launch{'es' if rec['launches'] > 1 else ''}, "
                f"{rec['kernel']}, {bshape.split_tokens}-token splits): {bus:.2f} us ({gbs(bbytes, bus):.0f} GB/s, "
                f"{rec['pct_of_peak']:.1f}% of peak); modes {rec['us_by_mode']}")
            del bt, bsc, bm, bl, bn, bo, bcnt
            torch.cuda.empty_cache()

    # ---- the reference's dense MMA geometry (attention_mma_supported: 8 query
    # rows sharing the KV, 24 q / 4 kv heads = group 6, dim 256, page 32) at
    # 65536 tokens: launch_attention_mma (its 256-token splits + merge), and
    # kvb_decode_attention at 1024-token splits.  KV bytes per call 136,314,880,
    # the byte count of the reference's own 64K benchmark
    # (data/att-bench-65536-v2-07.json).
    mma = None
    if not args.no_mma_geometry:
        mcaches = [W.torch_cache(8, 24, 4, 256, 32, 65536, seed=0x4B56440 + c, device="cuda:0")
                   for c in range(copies)]
        ms_ = mcaches[0][0]
        assert kvb.attention_mma_supported(ms_)
        minps = [kvb.device_input(t_["q"], t_["qpos"], t_["kpos"], t_["table"], t_["k"], t_["v"], t_["ks"], t_["vs"])
                 for _, t_ in mcaches]
        mrh = ms_.rows * ms_.q_heads
        msc = torch.empty(kvb.scratch_elements(ms_), dtype=torch.float32, device=dev)
        mm_, ml_ = torch.empty(mrh, device=dev), torch.empty(mrh, device=dev)
        mn_ = torch.empty(mrh * ms_.dim, device=dev)
        mbytes = 65536 * ms_.kv_heads * (2 * ms_.dim + 8)
        dst_ = 1024
        mma = {"shape": "8 rows x 24 q / 4 kv heads, dim 256, page 32, 65536 tokens",
               "kv_bytes_per_call": mbytes}
        mref = None
        if gate:
            t0_ = mcaches[0][1]
            mcase = W.Case(ms_, t0_["q"].cpu().numpy(), t0_["qpos"].cpu().numpy(), t0_["kpos"].cpu().numpy(),
                           t0_["table"].cpu().numpy().view(np.uint32), t0_["k"].cpu().numpy(),
                           t0_["v"].cpu().numpy(), t0_["ks"].cpu().numpy(), t0_["vs"].cpu().numpy())
            mref, _ = O.fp64(mcase, threads=host_threads)
            del mcase

        def mgate(label):
            o_, _, ok_ = O.normalize(mm_.cpu().numpy(), ml_.cpu().numpy(), mn_.cpu().numpy(), ms_.dim)
            g_ = O.gates(o_, mref)
            res = {"oracle": "fp64", "max_abs": g_["max_abs"], "rel_l2": g_["rel_l2"], "pass": bool(g_["pass"]),
                   "strict_3e-6+5e-5": bool(g_["strict_pass"])}
            log(f"gate {label}: {res}")
            if not ok_ or not g_["pass"]:
                fail(f"parity failed: {label}", parity=res)
            return res

        for key, fn_, nspl in (
                ("launch_attention_mma", lambda i: kvb.launch_attention_mma(ms_, minps[i % copies], msc, mm_, ml_, mn_,
                                                                            sp), kvb.split_count(ms_)),
                ("decode_1024_token_splits", lambda i: kvb.decode_attention(ms_, minps[i % copies], dst_, msc, mm_,
                                                                            ml_, mn_, stream=sp),
                 kvb.split_count(ms_, dst_))):
            if args.mma_calls not in ("both", key):
                continue
            rec = {"splits": nspl}
            fn_(0)
            torch.cuda.synchronize()
            if gate:
                rec["parity"] = mgate(f"mma geometry {key} (copy 0)")
            b0 = bits(mn_)
            mus = warm_and_time(fn_, steps=max(50, args.steps // 4), warmup=10) * 1e3
            fn_(0)
            torch.cuda.synchronize()
            if not np.array_equal(b0, bits(mn_)):
                fail(f"mma geometry {key}: output changed between calls (repeat check)")
            rec.update({"us_per_call": round(mus, 3), "GB/s": round(gbs(mbytes, mus), 1),
                        "pct_of_peak": round(100.0 * gbs(mbytes, mus) / HBM_PEAK_GBS, 2),
                        "kernel": kvb.selected_kernel_name(ms_, minps[0], 256 if key == "launch_attention_mma" else dst_),
                        "repeat_bitwise": True})
            mma[key] = rec
            log(f"mma geometry ({key}, {nspl} splits): {mus:.2f} us ({gbs(mbytes, mus):.0f} GB/s, "
                f"{rec['pct_of_peak']:.1f}% of peak)")
        if args.mma_calls == "both":
            # The same K, V and scale bytes through the same page table (two
            # 32-token pages per 64-token tile) with the 1,024-token work split
            # and no arithmetic: the read floor of this access pattern.
            msink = torch.zeros(kvb.split_count(ms_, dst_) * ms_.kv_heads, dtype=torch.int32, device=dev)
            pus = warm_and_time(lambda i: kvb.paged_read_probe(ms_, minps[i % copies], dst_, msink, sp),
                                steps=max(50, args.steps // 4), warmup=10) * 1e3
            mma["paged_probe_1024_token_splits"] = {
                "us": round(pus, 3), "GB/s": round(gbs(mbytes, pus), 1),
                "pct_of_peak": round(100.0 * gbs(mbytes, pus) / HBM_PEAK_GBS, 2),
                "note": "the geometry's own K, V and scale bytes through its page table, 1024-token work split, "
                        "no arithmetic (kvb_paged_read_probe)"}
            log(f"mma geometry paged probe (1024-token splits): {pus:.2f} us ({gbs(mbytes, pus):.0f} GB/s, "
                f"{mma['paged_probe_1024_token_splits']['pct_of_peak']:.1f}% of peak)")
        del mcaches, minps, msc
        torch.cuda.empty_cache()

    # ---- known-size kernels for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE
    if args.calibrate:
        cal_bytes = 256 << 20
        src = torch.empty(cal_bytes, dtype=torch.uint8, device=dev)
        dst = torch.empty(cal_bytes, dtype=torch.uint8, device=dev)
        for _ in range(5):
            dst.copy_(src)                                   # reads and writes cal_bytes
            kvb.hbm_read_probe(src, cal_bytes, sink, n_cu)   # reads cal_bytes
        torch.cuda.synchronize()
        log(f"calibration: 5 x copy of {cal_bytes} B and 5 x read probe of {cal_bytes} B")

    # ---- HBM traffic per launch of the benchmarked kernel, from committed rocprofv3 counter runs
    traffic = None
    tpath = os.path.join(root, "profiles", "traffic_cfg2.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            tinfo = json.load(fh)
        if tinfo.get("kernel") == fused_kernel:
            traffic = tinfo.get("hbm_bytes_per_launch")

    # ---- CPU baselines on this host: the reference's FP64 oracle (scalar,
    # one core) at cfg2 and cfg1, and a threaded fp32 split-K + LSE merge
    # restatement (attention_shared.cu:42-209, :295-335) at cfg1 and cfg2.
    cpu, cpu_more = None, None
    if not args.no_cpu_baseline and gate:
        kind = "reference" if O.ref_available() else "port"
        fn64 = O.ref_fp64 if kind == "reference" else (lambda c: O.fp64(c, threads=1))

        def median_time(fn, budget, min_runs=3, max_runs=50):
            times = []
            t_start = time.perf_counter()
            while len(times) < min_runs or (time.perf_counter() - t_start < budget and len(times) < max_runs):
                t0 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t0)
            return statistics.median(times), len(times)

        case2, _ = fp64_ref(0)
        med, runs = median_time(lambda: fn64(case2), args.cpu_seconds)
        cpu = {"value": kv_bytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": kind, "us_per_call": med * 1e6,
               "sample": f"{runs} full cfg2 calls (FP64 scalar oracle, examples/attention_reference.h), median",
               "host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
        log(f"cpu baseline ({kind}, FP64, 1 core): {med*1e3:.1f} ms/call at cfg2")
        nthreads = args.cpu_threads or len(os.sched_getaffinity(0))
        case1, st1 = W.cfg1()
        cpu_more = {"host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
        med1, runs1 = median_time(lambda: fn64(case1), 2.0, min_runs=5, max_runs=200)
        cfg1_bytes = case1.shape.tokens * case1.shape.kv_heads * (2 * case1.shape.dim + 8)
        cpu_more["fp64_cfg1"] = {"us_per_call": round(med1 * 1e6, 2), "cores": 1, "kind": kind, "runs": runs1,
                                 "GB/s": round(cfg1_bytes / med1 / 1e9, 4)}

        def split_merge(case, st_):
            sc_, ns_ = O.split_fp32(case, st_, threads=nthreads)
            return O.merge_fp32(case.shape, sc_, ns_)

        for label, case_, st_, kvb_bytes, budget in (("fp32_split_merge_cfg1", case1, st1, cfg1_bytes, 2.0),
                                                    ("fp32_split_merge_cfg2", case2, st, kv_bytes, 8.0)):
            med_, runs_ = median_time(lambda: split_merge(case_, st_), budget, min_runs=5, max_runs=200)
            cpu_more[label] = {"us_per_call": round(med_ * 1e6, 2), "cores": nthreads, "kind": "port", "runs": runs_,
                               "GB/s": round(kvb_bytes / med_ / 1e9, 4)}
            log(f"cpu {label} ({nthreads} threads): {med_*1e3:.2f} ms/call")

    call_ms = eager_ms
    value = gbs(kv_bytes, call_ms * 1e3)
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
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic",
        "config": {"workload": "cfg2: 1 seq, 32q/8kv heads, d128, 65536 tokens, page 64, random 1024-page "
                               "permutation, int8 KV + per-(token,kv_head) fp32 scales, 32 splits, fp16 out",
                   "kv_copies_rotated": copies, "kv_bytes_per_call": kv_bytes, "split_tokens": st,
                   "splits": splits},
        "timing": {"settle_seconds": args.settle_seconds, "settle_calls": settle_calls,
                   "graph_packet_capture_env": os.environ.get("DEBUG_CLR_GRAPH_PACKET_CAPTURE"),
                   "method": "back-to-back calls, HIP events on the launch stream; one untimed call queued "
                             "before the start event of every timed section (graph legs: >= 64 replays)",
                   "per_call_events_us": {"p50": round(p50, 3), "p95": round(p95, 3), "min": round(per_iter[0], 3),
                                          "warmup": 8, "iters": 32},
                   "repeat_bitwise": repeat_ok},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": fused_kernel, "algorithmic_bytes_per_launch": kv_bytes,
                     "launch_us": round(call_ms * 1e3, 3)},
        "two_launch": two,
        "fused_fenced": fenced,
        "launch_attention_256_token_splits": ref_api,
        "graph": graph,
        "split_only": {"kernel": split_kernel, "us": round(split_ms * 1e3, 3),
                       "GB/s": round(gbs(kv_bytes, split_ms * 1e3), 1)},
        "merge_only_us": round(merge_ms * 1e3, 3),
        "stream_probe": {"bytes": kv_bytes, "us": round(probe_ms * 1e3, 3), "GB/s": round(gbs(kv_bytes, probe_ms * 1e3), 1),
                         "pct_of_peak": round(100.0 * gbs(kv_bytes, probe_ms * 1e3) / HBM_PEAK_GBS, 2),
                         "note": "one contiguous streaming-read launch of the call's KV byte count, rotated buffers"},
        "stream_probe_paged": {"bytes": kv_bytes, "us": round(paged_ms * 1e3, 3),
                               "GB/s": round(gbs(kv_bytes, paged_ms * 1e3), 1),
                               "pct_of_peak": round(100.0 * gbs(kv_bytes, paged_ms * 1e3) / HBM_PEAK_GBS, 2),
                               "note": "the call's own K, V and scale bytes through its page table, decode work "
                                       "split, no arithmetic (kvb_paged_read_probe)"},
        "five_layer_step": five,
        "batched": batched,
        "mma_geometry": mma,
        "append": append,
        "cpu_baseline": cpu,
        "cpu_baselines_more": cpu_more,
        "parity": parity,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
