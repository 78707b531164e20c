"""Batched ragged decode (kvb_decode_attention_batched) on the GPU.

Every sequence of a batch must give exactly (bitwise) what a single-sequence
call on the same data gives -- the batched kernels only rebase pointers per
sequence, and splits past a sequence's own count hold empty partials that
every merge skips -- and must pass the north-star gate against the FP64
oracle.  BASELINE configs[2] (16 ragged sequences, 1K..32K tokens, shared
shuffled pool) and configs[3] (4 x 131072 tokens, GQA 8, 1% outlier tokens,
64 splits) run at full size.  A captured graph is replayed with the device
lengths changed between replays."""
import zlib

import numpy as np
import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import DeviceCase, check_against_oracle, log

pytestmark = pytest.mark.gpu


class DeviceBatch:
    def __init__(self, shape, t, device="cuda:0"):
        import torch

        self.shape, self.t, self.device = shape, t, device
        self.inp = kvb.batch_input(t["q"], t["qpos"], t["starts"], t["offsets"], t["kpos"], t["table"], t["k"],
                                   t["v"], t["ks"], t["vs"])
        rh = kvb.batch_output_scalar_elements(shape)
        self.rh = rh
        self.m = torch.empty(rh, dtype=torch.float32, device=device)
        self.l = torch.empty(rh, dtype=torch.float32, device=device)
        self.n = torch.empty(rh * shape.dim, dtype=torch.float32, device=device)
        self.scratch = torch.full((kvb.batch_scratch_elements(shape),), float("nan"), dtype=torch.float32,
                                  device=device)
        self.counters = torch.zeros(shape.batch * shape.kv_heads, dtype=torch.int32, device=device)

    def run(self, fused, out_type=kvb.KVB_OUT_F32):
        import torch

        dt = torch.float16 if out_type == kvb.KVB_OUT_F16 else torch.float32
        out = torch.full((self.rh * self.shape.dim,), float("nan"), dtype=dt, device=self.device)
        kvb.decode_attention_batched(self.shape, self.inp, self.scratch, self.m, self.l, self.n, out, out_type,
                                     counters=self.counters if fused else None)
        torch.cuda.synchronize()
        if fused:
            assert torch.count_nonzero(self.counters).item() == 0, "counters not left zero"
        return (self.m.cpu().numpy().copy(), self.l.cpu().numpy().copy(), self.n.cpu().numpy().copy(),
                out.float().cpu().numpy().reshape(self.rh, self.shape.dim))


def seq_slice(bc_shape, b):
    rh = bc_shape.rows * bc_shape.q_heads
    return slice(b * rh, (b + 1) * rh)


def check_sequence_vs_oracle(bc, b, m, l, n, label, threads=8):
    s = bc.shape
    sl = seq_slice(s, b)
    if bc.lengths[b] == 0:
        assert np.all(np.isneginf(m[sl])) and np.all(l[sl] == 0) and np.all(n.reshape(-1, s.dim)[sl] == 0), label
        return None
    case = bc.sequence(b)
    return check_against_oracle(case, (m[sl], l[sl], n.reshape(-1, s.dim)[sl].ravel()), label,
                                O.fp64(case, threads=threads))


BATCHES = [
    # rows, q_heads, kv_heads, dim, page, lengths, split_tokens
    (1, 32, 8, 128, 64, [100, 0, 4097, 64, 1, 2048, 777], 1024),   # ragged incl. empty, cfg2/3 geometry
    (2, 16, 4, 128, 64, [513, 1000, 64], 256),                     # 8 head-rows (two rows share KV)
    (1, 64, 8, 128, 64, [3000, 65, 1500], 512),                    # GQA 8
    (1, 8, 2, 64, 64, [300, 129, 0, 1], 64),                       # dim 64
    (1, 4, 4, 256, 64, [700, 70], 256),                            # dim 256
    (1, 8, 2, 64, 16, [300, 50, 0], 64),                           # page 16: generic batched kernel
    (1, 32, 8, 128, 64, [40000, 12000], 2048),                     # 20 + 6 splits of a 20-split stride
]


@pytest.mark.parametrize("cfg", BATCHES)
def test_batched_equals_single_calls_and_oracle(gpu, cfg):
    import torch

    rows, qh, kvh, d, p, lengths, st = cfg
    seed = zlib.crc32(repr(cfg).encode()) & 0xFFFF
    bc = W.synth_batch(rows, qh, kvh, d, p, lengths, seed=seed, split_tokens=st)
    db = DeviceBatch(bc.shape, bc.to_device("cuda:0"))
    log(f"batched shape={bc.shape.as_tuple()} lengths={lengths} kernel={kvb.batch_kernel_name(bc.shape, db.inp)} "
        f"fused kernel={kvb.batch_kernel_name(bc.shape, db.inp, fused=True)}")
    two = db.run(fused=False)
    fus = db.run(fused=True)
    batched_i8 = kvb.batch_kernel_name(bc.shape, db.inp).startswith("split_i8_kernel")

    def same(a, b_, what):
        if batched_i8:  # same kernel as the single call: bitwise
            assert np.array_equal(a, b_), what
        else:
            # generic fp32 batched kernel vs the int8-MFMA single-call kernel:
            # different arithmetic (the int8 kernel rounds the weights to 20
            # bits per chunk), both already gated against FP64 above; here
            # they must agree to 5e-5 of the largest magnitude.
            fin = np.isfinite(b_)
            assert np.array_equal(np.isfinite(a), fin), what
            scale_ = max(1.0, float(np.abs(b_[fin]).max(initial=0)))
            np.testing.assert_allclose(a[fin], b_[fin], rtol=0, atol=5e-5 * scale_, err_msg=what)

    for b, T in enumerate(bc.lengths):
        sl = seq_slice(bc.shape, b)
        check_sequence_vs_oracle(bc, b, *fus[:3], f"seq {b} (T={T}) fused")
        if T == 0:
            continue
        case = bc.sequence(b)
        dc = DeviceCase(case)
        # two-launch single call vs the two-launch batched call
        (m1, l1, n1), out1, _ = dc.run_decode(st)
        same(two[0][sl], m1, f"seq {b}: m differs")
        same(two[1][sl], l1, f"seq {b}: l differs")
        same(two[2].reshape(-1, d)[sl].ravel(), n1, f"seq {b}: n differs")
        same(two[3][sl], out1, f"seq {b}: out differs")
        # fused single call vs the fused batched call
        counters = torch.zeros(kvh, dtype=torch.int32, device=gpu)
        sc = dc.scratch(st)
        out = torch.full((rows * qh * d,), float("nan"), dtype=torch.float32, device=gpu)
        kvb.decode_attention_fused(case.shape, dc.inp, st, sc, counters, dc.m, dc.l, dc.n, out, kvb.KVB_OUT_F32)
        torch.cuda.synchronize()
        m2, l2, n2 = dc.read()
        same(fus[0][sl], m2, f"seq {b}: fused m differs")
        same(fus[1][sl], l2, f"seq {b}: fused l differs")
        same(fus[2].reshape(-1, d)[sl].ravel(), n2, f"seq {b}: fused n differs")
        same(fus[3][sl], out.cpu().numpy().reshape(-1, d), f"seq {b}: fused out differs")


def _full_config(gpu, cfg, lengths, seed, label):
    """Full-size config through the single-launch batched call: the fp32
    output passes the north-star gate against FP64 for every sequence; the
    fp16 output is that fp32 output rounded to nearest (bitwise), its own
    gate against FP64 is reported (fp16 cannot hold 2e-3 absolute once
    |out| > 4, which the 8x outlier tokens of configs[3] produce)."""
    import torch

    shape, t, lengths = W.torch_batch(cfg["rows"], cfg["q_heads"], cfg["kv_heads"], cfg["dim"],
                                      cfg["page_tokens"], lengths, seed=seed, split_tokens=cfg["split_tokens"],
                                      outlier_frac=cfg.get("outlier_frac", 0.0))
    torch.cuda.synchronize()
    db = DeviceBatch(shape, t)
    log(f"{label}: shape={shape.as_tuple()} splits/seq={kvb.batch_split_count(shape)} "
        f"kernel={kvb.batch_kernel_name(shape, db.inp, fused=True)} tokens={sum(lengths)}")
    m, l, n, out32 = db.run(fused=True, out_type=kvb.KVB_OUT_F32)
    out16 = db.run(fused=True, out_type=kvb.KVB_OUT_F16)[3]
    m2, l2, n2, _ = db.run(fused=False)
    assert np.array_equal(out16, out32.astype(np.float16).astype(np.float32)), "fp16 output != rounded fp32 output"
    bc = W.batch_to_host(shape, t, lengths)
    del t
    for b, T in enumerate(lengths):
        sl = seq_slice(shape, b)
        case = bc.sequence(b)
        ref = O.fp64(case, threads=16)
        check_against_oracle(case, (m[sl], l[sl], n.reshape(-1, shape.dim)[sl].ravel()), f"{label} seq {b} T={T}",
                             ref)
        g32 = O.gates(out32[sl], ref[0])
        g16 = O.gates(out16[sl], ref[0])
        log(f"  {label} seq {b}: fp32 out max_abs={g32['max_abs']:.2e} rel_l2={g32['rel_l2']:.2e}; "
            f"fp16 out max_abs={g16['max_abs']:.2e} rel_l2={g16['rel_l2']:.2e} max|out|={np.abs(ref[0]).max():.2f}")
        assert g32["pass"], g32
        assert g16["rel_l2"] <= 1e-3, g16
        assert np.array_equal(m[sl], m2[sl])
        np.testing.assert_allclose(l[sl], l2[sl], rtol=3e-6, atol=0)


def test_cfg3_ragged_batch_full(gpu):
    """16 sequences, lengths uniform in [1024, 32768]."""
    _full_config(gpu, W.CFG3, W.cfg3_lengths(), 0x4B56423, "cfg3")


def test_cfg4_wide_gqa_full(gpu):
    """4 x 131072 tokens, 64q/8kv, 1% outlier tokens, 64 splits."""
    cfg = dict(W.CFG4)
    _full_config(gpu, cfg, cfg.pop("lengths"), 0x4B56424, "cfg4")


def test_batched_graph_replay_with_changing_lengths(gpu):
    """One captured batched call replayed while the device-side lengths change;
    each replay equals an eager call on the same metadata."""
    import torch

    lengths = [3000, 1200, 64, 2500]
    bc = W.synth_batch(1, 32, 8, 128, 64, lengths, seed=77, split_tokens=512)
    t = bc.to_device("cuda:0")
    db = DeviceBatch(bc.shape, t)
    starts_host = bc.seq_starts.astype(np.int64)
    variants = []
    for shrink in ([0, 0, 0, 0], [500, 1199, 0, 2499], [2999, 0, 63, 100]):
        # shorten sequence b to its first T_b - shrink_b tokens (same pages, same positions)
        st = np.array(starts_host)
        new_starts = [0]
        kpos = []
        for b, T in enumerate(lengths):
            T2 = T - shrink[b]
            kpos.append(bc.kpos[st[b]:st[b] + T2])
            new_starts.append(new_starts[-1] + T2)
        variants.append((np.array(new_starts, np.uint32), np.concatenate(kpos), [T - s for T, s in zip(lengths, shrink)]))
    qpos_t = t["qpos"]
    kpos_t = torch.zeros_like(t["kpos"])
    starts_t = torch.zeros_like(t["starts"])
    db.inp = kvb.batch_input(t["q"], qpos_t, starts_t, t["offsets"], kpos_t, t["table"], t["k"], t["v"], t["ks"],
                             t["vs"])

    def load_variant(v):
        starts, kpos, lens = v
        starts_t.copy_(torch.from_numpy(starts.view(np.int32)))
        kpos_t.zero_()
        kpos_t[:len(kpos)].copy_(torch.from_numpy(kpos))
        qpos_t.copy_(torch.tensor([T - 1 for T in lens], dtype=torch.int64))

    eager = []
    for v in variants:
        load_variant(v)
        torch.cuda.synchronize()
        eager.append(db.run(fused=True, out_type=kvb.KVB_OUT_F16)[3].copy())
    out = torch.zeros(db.rh * 128, dtype=torch.float16, device=gpu)
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()  # `out` was filled on the default stream
    with torch.cuda.stream(stream):  # warm-up on the capture stream
        kvb.decode_attention_batched(bc.shape, db.inp, db.scratch, db.m, db.l, db.n, out, kvb.KVB_OUT_F16,
                                     counters=db.counters, stream=stream.cuda_stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=stream):
        kvb.decode_attention_batched(bc.shape, db.inp, db.scratch, db.m, db.l, db.n, out, kvb.KVB_OUT_F16,
                                     counters=db.counters, stream=stream.cuda_stream)
    for rep in range(2):
        for i, v in enumerate(variants):
            load_variant(v)
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = out.float().cpu().numpy().reshape(db.rh, 128)
            assert np.array_equal(got, eager[i]), f"replay {rep} variant {i} differs from eager"
            assert torch.count_nonzero(db.counters).item() == 0
        log(f"  graph replay {rep}: {len(variants)} length variants equal eager")
    # and the variants differ from each other (the replay really saw the new lengths)
    assert not np.array_equal(eager[0], eager[1]) and not np.array_equal(eager[1], eager[2])
