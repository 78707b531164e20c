"""Single-launch decode (kvb_decode_attention_fused): the last work-group of
each kv head merges the splits.  Checked against the FP64 oracle (north-star
gate), against the two-launch kvb_decode_attention (same partials, merge in a
different fp32 summation order), for the counters being left zero after every
call, for back-to-back calls on different inputs, and inside a replayed
hipGraph."""
import zlib

import numpy as np
import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import DeviceCase, check_against_oracle, log

pytestmark = pytest.mark.gpu


def run_fused(dc, split_tokens, counters, out_type=kvb.KVB_OUT_F32):
    import torch

    s = dc.case.shape
    rh = s.rows * s.q_heads
    sc = dc.scratch(split_tokens)
    dt = torch.float16 if out_type == kvb.KVB_OUT_F16 else torch.float32
    out = torch.full((rh * s.dim,), float("nan"), dtype=dt, device=dc.device)
    kvb.decode_attention_fused(s, dc.inp, split_tokens, sc, counters, dc.m, dc.l, dc.n, out, out_type)
    torch.cuda.synchronize()
    return dc.read(), out.float().cpu().numpy().reshape(rh, s.dim)


FUSED_SHAPES = [
    # rows, q_heads, kv_heads, dim, P, tokens, begin, end, split_tokens, qpos
    (1, 8, 2, 64, 16, 512, 0, 512, 128, None),          # cfg1 geometry
    (1, 32, 8, 128, 64, 8192, 0, 8192, 2048, None),     # cfg2 geometry, shorter
    (1, 32, 8, 128, 64, 3000, 100, 2900, 256, [1500]),  # causal cut inside the range
    (2, 16, 4, 128, 32, 1000, 37, 990, 64, [500, 990]),
    (1, 64, 8, 128, 64, 4096, 0, 4096, 1024, None),     # group 8
    (1, 4, 4, 256, 64, 1111, 0, 1111, 512, None),       # dim 256
    (1, 8, 2, 64, 16, 300, 0, 300, 64, [-1]),           # every row-head empty
    (8, 48, 8, 128, 64, 640, 64, 640, 256, None),       # 48 head-rows: two-launch fallback
    (1, 8, 2, 64, 16, 4096, 0, 4096, 64, None),         # 64 splits: merge in two chunks
    (1, 32, 8, 128, 64, 8192, 5, 8192, 64, [6000]),     # 128 splits, causal cut, ragged begin
    (2, 8, 2, 128, 32, 2000, 0, 2000, 32, [1999, 700]), # 8 head-rows, 63 splits
    (1, 32, 8, 128, 64, 4096, 0, 4096, 256, None),      # four-wave groups: one 16-split merge pass
    (1, 64, 8, 128, 64, 8192, 0, 8192, 256, [6000]),    # 8 head-rows, 32 splits: two 16-split merge passes
]


@pytest.mark.parametrize("cfg", FUSED_SHAPES)
def test_fused_matches_oracle_and_two_launch(gpu, cfg):
    import torch

    rows, qh, kvh, d, p, t, b, e, st, qpos = cfg
    case = W.synth_case(rows, qh, kvh, d, p, t, seed=zlib.crc32(repr(cfg).encode()) & 0xFFFF, begin=b, end=e, qpos=qpos)
    dc = DeviceCase(case)
    log(f"fused shape={case.shape.as_tuple()} split_tokens={st} "
        f"kernel={kvb.selected_kernel_name(case.shape, dc.inp, st, True)}")
    counters = torch.zeros(kvh, dtype=torch.int32, device=gpu)
    ref = O.fp64(case, threads=8)
    mln, out = run_fused(dc, st, counters)
    check_against_oracle(case, mln, "fused m/l/n", ref, strict=True)
    assert torch.count_nonzero(counters).item() == 0, "counters not left zero"
    (m2, l2, n2), out2, _ = dc.run_decode(st)
    m, l, n = mln
    assert np.array_equal(np.isneginf(m), np.isneginf(m2))
    fin = np.isfinite(m)
    assert np.array_equal(m[fin], m2[fin])
    np.testing.assert_allclose(l, l2, rtol=3e-6, atol=0)
    np.testing.assert_allclose(n, n2, rtol=3e-5, atol=3e-6 * max(1.0, float(np.abs(n2).max(initial=0))))
    np.testing.assert_allclose(out, out2, rtol=3e-5, atol=1e-6)


def test_fused_back_to_back_and_graph(gpu):
    """Two different caches alternately through one counters buffer, eagerly
    and replayed in a captured graph; every result checked."""
    import torch

    cases = [W.synth_case(1, 32, 8, 128, 64, 4096, seed=40 + i) for i in range(2)]
    dcs = [DeviceCase(c) for c in cases]
    refs = [O.fp64(c, threads=8) for c in cases]
    counters = torch.zeros(8, dtype=torch.int32, device=gpu)
    st = 512
    for rep in range(3):
        for dc, ref in zip(dcs, refs):
            mln, _ = run_fused(dc, st, counters)
            check_against_oracle(dc.case, mln, f"fused eager rep{rep}", ref)
            assert torch.count_nonzero(counters).item() == 0
    # graph: both calls captured once, replayed several times with eager work between
    s = cases[0].shape
    scs = [dc.scratch(st) for dc in dcs]
    outs = [torch.zeros(32 * 128, dtype=torch.float16, device=gpu) for _ in dcs]
    g = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()  # buffers above were filled on the default stream
    with torch.cuda.stream(stream):
        for dc, sc, o in zip(dcs, scs, outs):
            kvb.decode_attention_fused(s, dc.inp, st, sc, counters, dc.m, dc.l, dc.n, o, kvb.KVB_OUT_F16,
                                       stream.cuda_stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=stream):
        for dc, sc, o in zip(dcs, scs, outs):
            kvb.decode_attention_fused(s, dc.inp, st, sc, counters, dc.m, dc.l, dc.n, o, kvb.KVB_OUT_F16,
                                       stream.cuda_stream)
    for rep in range(4):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for dc, o, ref in zip(dcs, outs, refs):
            got = o.float().cpu().numpy().reshape(32, 128)
            gate = O.gates(got, ref[0])
            log(f"  graph replay {rep}: max_abs={gate['max_abs']:.2e} rel_l2={gate['rel_l2']:.2e}")
            assert gate["pass"], gate
        assert torch.count_nonzero(counters).item() == 0


def test_fused_rejects_null_counters(gpu):
    case, st = W.cfg1()
    dc = DeviceCase(case)
    with pytest.raises(kvb.KvbInvalidArgument, match="counters"):
        kvb.decode_attention_fused(case.shape, dc.inp, st, dc.scratch(st), None, dc.m, dc.l, dc.n)


def test_fenced_diagnostic_matches_fused(gpu):
    # kvb_decode_attention_fused_fenced: the same single launch with formal
    # release / acquire fences around the merge ticket.  Only the ordering
    # instructions differ, so m, l, n and the fp16 output are bitwise those of
    # the default call; shapes without an instance are rejected.
    import torch

    case = W.synth_case(1, 32, 8, 128, 64, 16384, seed=91, qpos=[12000])
    dc = DeviceCase(case)
    st = 1024  # 16 splits of 16 tiles: the eight-wave configuration
    assert kvb.selected_kernel_name(case.shape, dc.inp, st, True) == "split_i8_kernel<128,8,2,true,4,true,false,false>"
    s = case.shape
    rh = s.rows * s.q_heads
    res = []
    for fn in (kvb.decode_attention_fused, kvb.decode_attention_fused_fenced):
        counters = torch.zeros(s.kv_heads, dtype=torch.int32, device=dc.device)
        out = torch.full((rh * s.dim,), float("nan"), dtype=torch.float16, device=dc.device)
        for t in (dc.m, dc.l, dc.n):
            t.fill_(float("nan"))
        fn(s, dc.inp, st, dc.scratch(st), counters, dc.m, dc.l, dc.n, out, kvb.KVB_OUT_F16)
        torch.cuda.synchronize()
        assert torch.count_nonzero(counters).item() == 0
        res.append(dc.read() + (out.view(torch.int16).cpu().numpy().copy(),))
    for x, y, nm in zip(res[0], res[1], ("m", "l", "n", "out")):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"fenced call: {nm} differs"
    check_against_oracle(case, res[1][:3], "fenced single launch", strict=True)
    with pytest.raises(kvb.KvbInvalidArgument, match="fenced diagnostic"):
        small = W.synth_case(1, 8, 2, 64, 16, 512, seed=92)
        dcs = DeviceCase(small)
        kvb.decode_attention_fused_fenced(small.shape, dcs.inp, 128, dcs.scratch(128),
                                          torch.zeros(2, dtype=torch.int32, device=dcs.device),
                                          dcs.m, dcs.l, dcs.n, None, kvb.KVB_OUT_NONE)
