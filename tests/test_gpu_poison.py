"""GPU guard tests: every cache slot a call must not read is poisoned (K code
127, V code -128, k/v scales 1e4 -- tests/helpers.poison_unneeded: tokens in
the future of every query row, tokens before begin, slots past end in a
partial last page, unmapped pool pages), and the raw m, l, n of the call must
stay bitwise equal to the unpoisoned call's.  The reference's oracle test
does this for future tokens on the CPU (tests/reference_test.cpp:21-30);
here it runs through the split kernels' own masking: the int8 split kernel
(single launch, two launches, the one-wave form behind launch_attention),
the dense rows kernel behind launch_attention_mma and the decode call, and
the generic kernel.  The unpoisoned results are also gated against FP64."""
import numpy as np
import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import DeviceCase, check_against_oracle, log, poison_unneeded

pytestmark = pytest.mark.gpu


def _decode(dc, st):
    return dc.run_decode(st, kvb.KVB_OUT_F32)[0]


def _fused(dc, st):
    import torch

    s = dc.case.shape
    counters = torch.zeros(s.kv_heads, dtype=torch.int32, device=dc.device)
    out = torch.empty(s.rows * s.q_heads * s.dim, dtype=torch.float32, device=dc.device)
    kvb.decode_attention_fused(s, dc.inp, st, dc.scratch(st), counters, dc.m, dc.l, dc.n, out, kvb.KVB_OUT_F32)
    torch.cuda.synchronize()
    assert torch.count_nonzero(counters).item() == 0
    return dc.read()


def _reference_api(dc, st):
    return dc.run_reference_api(mma=False)[0]


def _mma(dc, st):
    return dc.run_reference_api(mma=True)[0]


CALLS = {"decode": _decode, "fused": _fused, "launch_attention": _reference_api, "launch_attention_mma": _mma}


def _check(case, st, calls, expect_kernel):
    pc, nbad = poison_unneeded(case)
    s = case.shape
    clean, dirty = DeviceCase(case), DeviceCase(pc)
    name = kvb.selected_kernel_name(s, clean.inp, st, fused=False)
    log(f"poison shape={s.as_tuple()} split_tokens={st} poisoned_slots={nbad} kernel={name}")
    assert expect_kernel in name, name
    ref = O.fp64(case, threads=8)
    for c in calls:
        a = CALLS[c](clean, st)
        b = CALLS[c](dirty, st)
        check_against_oracle(case, a, f"{c} (clean)", ref)
        for x, y, nm in zip(a, b, ("m", "l", "n")):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"{c}: poisoned slots changed {nm}"
        log(f"  {c}: m/l/n bitwise equal with {nbad} poisoned slots")


def test_poison_int8_cfg2_geometry_causal(gpu):
    # cfg2 geometry (32 q / 8 kv heads, dim 128, 64-token pages, random pages,
    # 4 spare pool pages), begin 100, partial last page (end 15977), query at
    # position 9000: everything after it is in the future.
    case = W.synth_case(1, 32, 8, 128, 64, 16384, seed=81, pages=260, begin=100, end=15977, qpos=[9000])
    _check(case, 2048, ["fused", "decode", "launch_attention"], "split_i8_kernel<128,")


def test_poison_int8_cfg2_geometry_partial_last_page(gpu):
    # Every token of [begin, end) visible; the poison sits before begin, past
    # end in the last page and in unmapped pages.
    case = W.synth_case(1, 32, 8, 128, 64, 16384, seed=82, pages=260, begin=64, end=16361, qpos=[20000])
    _check(case, 2048, ["fused", "decode", "launch_attention"], "split_i8_kernel<128,")


def test_poison_dense_rows_causal_self_test_shape(gpu):
    # The reference self-test's causal case (examples/attention_bench.cu:156-168,
    # query rows at 17 r) on the closed-form fixture, 513 tokens (partial last
    # page), through launch_attention_mma and launch_attention.
    f = O.fixture(513, permute=True)
    f.qpos = np.arange(8, dtype=np.int64) * 17
    _check(f, 256, ["launch_attention_mma", "launch_attention"], "split_i8_rows")


def test_poison_dense_rows_long(gpu):
    # Dense geometry over 4096 tokens, query rows at 2000 + 100 r: tokens
    # after 2700 are in every row's future; decode at 1024-token splits and
    # the reference's entry points.
    case = W.synth_case(8, 24, 4, 256, 32, 4096, seed=83, pages=130, begin=0, end=4090,
                        qpos=[2000 + 100 * r for r in range(8)])
    _check(case, 1024, ["decode", "launch_attention_mma"], "split_i8_rows")


def test_poison_generic_int8(gpu):
    case = W.synth_case(1, 8, 2, 96, 48, 1000, seed=84, pages=24, begin=37, end=950, qpos=[700])
    _check(case, 256, ["decode", "fused", "launch_attention"], "split_generic")


def test_poison_generic_fp32_kv(gpu):
    case = W.synth_case(1, 8, 2, 64, 16, 700, seed=85, pages=48, begin=10, end=650, qpos=[500], int8=False)
    _check(case, 128, ["decode", "launch_attention"], "split_generic")
