"""kvb_decode_attention_noalloc (the single-launch call with the library's own
fixed per-device scratch) against kvb_decode_attention_fused with caller
buffers: bitwise equal m, l, n and fp16 output on two calls in a row, the
second with a smaller input; counters of the caller-buffer call left zero;
an oversized call rejected before anything is enqueued."""
import numpy as np
import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import DeviceCase, check_against_oracle, log

pytestmark = pytest.mark.gpu


def _run(dc, st, noalloc):
    import torch

    s = dc.case.shape
    rh = s.rows * s.q_heads
    out = torch.full((rh * s.dim,), float("nan"), dtype=torch.float16, device=dc.device)
    for t in (dc.m, dc.l, dc.n):
        t.fill_(float("nan"))
    if noalloc:
        kvb.decode_attention_noalloc(s, dc.inp, st, dc.m, dc.l, dc.n, out, kvb.KVB_OUT_F16)
    else:
        counters = torch.zeros(s.kv_heads, dtype=torch.int32, device=dc.device)
        kvb.decode_attention_fused(s, dc.inp, st, dc.scratch(st), counters, dc.m, dc.l, dc.n, out, kvb.KVB_OUT_F16)
        torch.cuda.synchronize()
        assert torch.count_nonzero(counters).item() == 0
    torch.cuda.synchronize()
    m, l, n = dc.read()
    return m, l, n, out.view(torch.int16).cpu().numpy().copy()


def test_noalloc_matches_fused_two_calls(gpu):
    # First the cfg2 geometry (32 kv-head splits of 2048 tokens), then a
    # smaller cfg1-shaped call through the same static scratch.
    cases = [(W.synth_case(1, 32, 8, 128, 64, 16384, seed=71), 2048), W.cfg1()]
    for i, (case, st) in enumerate(cases):
        dc = DeviceCase(case)
        log(f"no-alloc call {i}: shape={case.shape.as_tuple()} split_tokens={st} "
            f"kernel={kvb.selected_kernel_name(case.shape, dc.inp, st, fused=True)}")
        a = _run(dc, st, noalloc=True)
        b = _run(dc, st, noalloc=False)
        for x, y, name in zip(a, b, ("m", "l", "n", "out")):
            assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"call {i}: {name} differs"
        check_against_oracle(case, a[:3], f"no-alloc call {i}", O.fp64(case, threads=8))


def test_noalloc_rejects_oversized_call(gpu):
    # 1 row x 64 q heads, 256-token splits over 1M tokens: 64 x 4096 x 130 floats > 8 MiB.
    s = kvb.make_shape(1, 64, 8, 128, 64, 16384, 1 << 20, 0, 1 << 20, 0.0883883)
    fake = 0x1000
    inp = kvb.device_input(fake, fake, fake, fake, fake, fake, fake, fake)
    with pytest.raises(kvb.KvbInvalidArgument, match="static area"):
        kvb.decode_attention_noalloc(s, inp, 256, fake, fake, fake, fake, kvb.KVB_OUT_F16)


def test_noalloc_kv_heads_across_counter_region(gpu):
    # Calls on both sides of 64 kv heads in a row through the one static
    # area: 8 kv heads, then a single-launch call with 128 kv heads (1 row,
    # 128 q heads, dim 128, 2 splits), then 8 again.  The counter words of
    # the wide call must not hold partial words of the first call, and its
    # partials must not land on counter words the third call needs at zero.
    cases = [(W.synth_case(1, 32, 8, 128, 64, 8192, seed=72), 2048),
             (W.synth_case(1, 128, 128, 128, 64, 2048, seed=73), 1024),
             (W.synth_case(1, 32, 8, 128, 64, 8192, seed=74), 2048)]
    for i, (case, st) in enumerate(cases):
        dc = DeviceCase(case)
        name = kvb.selected_kernel_name(case.shape, dc.inp, st, fused=True)
        log(f"no-alloc sequence call {i}: shape={case.shape.as_tuple()} split_tokens={st} kernel={name}")
        assert name.endswith(",true,false,false>"), f"call {i} is not a single launch: {name}"
        a = _run(dc, st, noalloc=True)
        b = _run(dc, st, noalloc=False)
        for x, y, nm in zip(a, b, ("m", "l", "n", "out")):
            assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"call {i}: {nm} differs"
        check_against_oracle(case, a[:3], f"no-alloc sequence call {i}", O.fp64(case, threads=8))
