"""Shared helpers for the GPU parity tests: run a Case through the C ABI and
compare with the CPU oracle."""
from __future__ import annotations

import sys

import numpy as np

import kvbridge_amd as kvb
from oracle import oracle as O


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


class DeviceCase:
    """Device copies of a Case plus caller-owned output buffers."""

    def __init__(self, case, device="cuda:0"):
        import torch

        self.case = case
        self.t = case.to_device(device)
        self.device = device
        t = self.t
        self.inp = kvb.device_input(t["q"], t["qpos"], t["kpos"], t["table"], t["k"], t["v"], t["ks"], t["vs"])
        s = case.shape
        rh = s.rows * s.q_heads
        self.m = torch.empty(rh, dtype=torch.float32, device=device)
        self.l = torch.empty(rh, dtype=torch.float32, device=device)
        self.n = torch.empty(rh * s.dim, dtype=torch.float32, device=device)

    def scratch(self, split_tokens=None):
        import torch

        return torch.full((kvb.scratch_elements(self.case.shape, split_tokens),), float("nan"),
                          dtype=torch.float32, device=self.device)

    def run_reference_api(self, mma=False, shape=None):
        import torch

        s = shape or self.case.shape
        sc = self.scratch()
        fn = kvb.launch_attention_mma if mma else kvb.launch_attention
        fn(s, self.inp, sc, self.m, self.l, self.n)
        torch.cuda.synchronize()
        return self.read(), sc

    def run_decode(self, split_tokens, out_type=kvb.KVB_OUT_F32, shape=None):
        import torch

        s = shape or self.case.shape
        sc = self.scratch(split_tokens)
        rh = s.rows * s.q_heads
        dt = torch.float16 if out_type == kvb.KVB_OUT_F16 else torch.float32
        out = torch.full((rh * s.dim,), float("nan"), dtype=dt, device=self.device)
        kvb.decode_attention(s, self.inp, split_tokens, sc, self.m, self.l, self.n, out, out_type)
        torch.cuda.synchronize()
        return self.read(), out.float().cpu().numpy().reshape(rh, s.dim), sc

    def read(self):
        return (self.m.cpu().numpy().copy(), self.l.cpu().numpy().copy(), self.n.cpu().numpy().copy())


def check_against_oracle(case, mln, label, ref=None, strict=False):
    """North-star gate on n/l against FP64 (asserted); the reference's
    per-element gate |a - r| <= 3e-6 + 5e-5|r| (examples/attention_bench.cu:127)
    is asserted too when strict, else reported."""
    s = case.shape
    m, l, n = mln
    out, vis, ok = O.normalize(m, l, n, s.dim)
    if ref is None:
        ref = O.fp64(case, threads=8)
    ref_out, ref_vis = ref
    assert ok, f"{label}: empty-row convention or finiteness violated"
    assert np.array_equal(vis, ref_vis), f"{label}: visibility differs ({vis.sum()} vs {ref_vis.sum()})"
    g = O.gates(out, ref_out)
    log(f"  {label}: max_abs={g['max_abs']:.3e} rel_l2={g['rel_l2']:.3e} strict={'PASS' if g['strict_pass'] else 'fail'}")
    assert g["pass"], f"{label}: {g}"
    if strict:
        assert g["strict_pass"], f"{label}: per-element gate 3e-6 + 5e-5|r| failed: {g}"
    return g


def poison_unneeded(case, k_code=127, v_code=-128, scale=1.0e4):
    """Copy of `case` with every cache slot the call must not read overwritten:
    K code 127, V code -128 (fp32 KV: K 127 * scale, V -128 * scale) and large
    finite k/v scales -- the future-poison idea of the reference's oracle test
    (tests/reference_test.cpp:21-30) applied to the whole pool.  A slot is
    needed only when it holds a logical token t of [begin, end) with
    k_positions[t] <= max(q_positions); every other slot is poisoned: tokens
    in the future of every query row, tokens before begin, slots past end in
    a partial last page, and physical pages no logical page of the range maps
    to.  Returns (poisoned case, number of poisoned (page, slot) pairs)."""
    import copy

    s = case.shape
    P = s.page_tokens
    need = np.zeros((s.pages, P), bool)
    qmax = int(np.max(case.qpos)) if s.rows > 0 else -1
    for t in range(s.begin, s.end):
        if int(case.kpos[t]) <= qmax:
            need[int(case.table[t // P]), t % P] = True
    bad = ~need
    c = copy.deepcopy(case)
    if s.int8:
        kk, vv = np.int8(k_code), np.int8(v_code)
    else:
        kk, vv = np.float32(k_code * scale), np.float32(v_code * scale)
    pg, sl = np.nonzero(bad)
    c.k[pg, :, sl, :] = kk
    c.v[pg, :, :, sl] = vv
    c.ks[pg, :, sl] = np.float32(scale)
    c.vs[pg, :, sl] = np.float32(scale)
    return c, int(bad.sum())
