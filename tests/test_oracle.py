"""The CPU oracle (oracle/attention_oracle.c) pinned before it is trusted.

Checks, each tied to what fixes the answer:
  * golden vectors in tests/golden, written by the reference's own FP64
    oracle (examples/attention_reference.h:53-90) built from source;
  * the reference's known-answer tests (tests/reference_test.cpp:7-37):
    zero-Q closed form (mean of causal V), page-permutation invariance,
    future-poison invariance, empty and fully masked intervals;
  * the closed-form fixture against the reference generator
    (examples/attention_reference.h:19-48) when oracle/_ref is built;
  * an independent dense numpy FP64 formulation on tiny shapes;
  * split + merge (fp32) against FP64 for any split size, the one-split
    identity and the all-empty convention (src/attention_shared.cu:295-335);
  * planted mistakes (oracle_set_fault): every one must fail a check above.
"""
import glob
import os

import numpy as np
import pytest

from kvbridge_amd import workloads as W
from kvbridge_amd._capi import Shape
from oracle import oracle as O

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def _shape_from(arr):
    a = [float(x) for x in arr]
    return Shape(*[int(x) for x in a[:9]], a[9], int(a[10]))


def load_golden(path):
    z = np.load(path, allow_pickle=False)
    shape = _shape_from(z["shape"])
    if "fixture_tokens" in z.files:
        case = O.fixture(int(z["fixture_tokens"]), permute=bool(z["fixture_permute"]))
        case.shape = shape
        case.qpos = z["qpos"]
        rh = z["row_heads"]
    else:
        case = W.Case(shape, z["q"], z["qpos"], z["kpos"], z["table"], z["k"], z["v"], z["ks"], z["vs"])
        rh = np.arange(shape.rows * shape.q_heads)
    return case, rh, z["out"], z["visible"]


def golden_ok(path, tol=1e-12):
    case, rh, out, vis = load_golden(path)
    got, gvis = O.fp64(case, threads=4)
    if not np.array_equal(gvis[rh], vis):
        return False
    scale = max(1.0, float(np.abs(out).max()) if out.size else 1.0)
    return bool(np.all(np.abs(got[rh] - out) <= tol * scale))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden_vectors(path):
    assert golden_ok(path)


def test_golden_set_present():
    names = {os.path.basename(p)[:-4] for p in GOLDEN}
    assert {"cfg1", "ragged_causal", "empty_range", "fixture_case0", "fixture_case6"} <= names


# ---- known-answer tests of tests/reference_test.cpp ------------------------

def zero_q_closed_form_ok():
    """Q = 0 makes every logit 0: the output is the plain mean of the visible
    V values (reference_test.cpp:7-17).  qpos = 2 leaves tokens 0, 1, 2."""
    f = O.fixture(64, permute=True)
    f.q = np.zeros_like(f.q)
    f.qpos = np.full(8, 2, np.int64)
    out, vis = O.fp64(f)
    if not vis.all():
        return False
    t = np.arange(3)[:, None, None]
    h = np.arange(24)[None, :, None]
    d = np.arange(256)[None, None, :]
    kv = h // 6
    code = ((t * 7 + kv * 13 + d * 5) % 256) - 128
    vscale = ((t * 3 + kv) % 5 + 1) / 512.0
    expect = (code * vscale).mean(axis=0)  # [24, 256]
    got = out.reshape(8, 24, 256)
    return bool(np.all(np.abs(got - expect[None]) < 1e-14))


def permutation_invariant_ok():
    a, _ = O.fp64(O.fixture(64))
    b, _ = O.fp64(O.fixture(64, permute=True))
    return bool(np.array_equal(a, b))


def future_poison_ok():
    f = O.fixture(64, permute=True)
    f.q = np.zeros_like(f.q)
    f.qpos = np.full(8, 2, np.int64)
    before, _ = O.fp64(f)
    k, v = f.k.copy(), f.v.copy()
    for t in range(3, 64):
        page, slot = f.table[t // 32], t % 32
        k[page, :, slot, :] = 127
        v[page, :, :, slot] = -128
    f.k, f.v = k, v
    after, _ = O.fp64(f)
    return bool(np.array_equal(before, after))


def empty_and_masked_ok():
    f = O.fixture(64, permute=True)
    f.shape = f.shape.copy(begin=f.shape.end)
    out, vis = O.fp64(f)
    if vis.any() or np.any(out != 0):
        return False
    f = O.fixture(64, permute=True)
    f.qpos = np.full(8, -1, np.int64)
    out, vis = O.fp64(f)
    return not vis.any()


def test_zero_q_closed_form():
    assert zero_q_closed_form_ok()


def test_page_permutation_invariance():
    assert permutation_invariant_ok()


def test_future_poison_invariance():
    assert future_poison_ok()


def test_empty_and_masked():
    assert empty_and_masked_ok()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("tokens,permute", [(64, False), (64, True), (256, True), (513, True)])
def test_fixture_matches_reference_generator(tokens, permute):
    mine = O.fixture(tokens, permute)
    ref = O.ref_fixture(tokens, permute)
    for a, b in zip((mine.q, mine.qpos, mine.kpos, mine.table, mine.k, mine.v, mine.ks, mine.vs), ref):
        assert np.array_equal(a, b)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_fp64_matches_reference_oracle_random(seed):
    rng = np.random.default_rng(seed)
    kv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 3, 4, 8]))
    P = int(rng.choice([16, 32, 48, 64]))
    D = int(rng.choice([8, 64, 128, 256]))
    T = int(rng.integers(50, 400))
    b = int(rng.integers(0, T // 3))
    e = int(rng.integers(b, T + 1))
    rows = int(rng.integers(1, 4))
    qpos = rng.integers(-2, T + 2, rows)
    case = W.synth_case(rows, kv * group, kv, D, P, T, seed=seed, begin=b, end=e, qpos=qpos)
    got, gvis = O.fp64(case, threads=4)
    ref, rvis = O.ref_fp64(case)
    assert np.array_equal(gvis, rvis)
    assert np.max(np.abs(got - ref), initial=0.0) <= 1e-12 * max(1.0, np.abs(ref).max(initial=0.0))


# ---- independent dense formulation -----------------------------------------

def dense_fp64(case):
    """Gather the paged cache into logical token order, dequantize, then
    softmax(Q K^T * scale) V per row-head with numpy (float64)."""
    s = case.shape
    group = s.q_heads // s.kv_heads
    t = np.arange(s.begin, s.end)
    page = case.table[t // s.page_tokens].astype(np.int64)
    slot = t % s.page_tokens
    ks = case.ks[page, :, slot] if s.int8 else np.ones((len(t), s.kv_heads))
    vs = case.vs[page, :, slot] if s.int8 else np.ones((len(t), s.kv_heads))
    k = case.k[page, :, slot, :].astype(np.float64) * ks[..., None]          # [T, kv, D]
    v = case.v[page, :, :, slot].astype(np.float64) * vs[..., None]          # [T, kv, D]
    q = case.q.reshape(s.rows, s.q_heads, s.dim).astype(np.float64)
    out = np.zeros((s.rows * s.q_heads, s.dim))
    vis = np.zeros(s.rows * s.q_heads, bool)
    for r in range(s.rows):
        mask = case.kpos[t] <= case.qpos[r]
        if not mask.any():
            continue
        for h in range(s.q_heads):
            kvh = h // group
            logits = (k[mask, kvh, :] @ q[r, h]) * np.float64(np.float32(s.scale))
            w = np.exp(logits - logits.max())
            out[r * s.q_heads + h] = (w @ v[mask, kvh, :]) / w.sum()
            vis[r * s.q_heads + h] = True
    return out, vis


@pytest.mark.parametrize("cfg", [
    (1, 4, 2, 16, 16, 70, 0, 70, False),
    (2, 6, 2, 32, 48, 130, 9, 121, True),
    (3, 8, 8, 8, 16, 40, 5, 40, True),
    (1, 4, 1, 64, 64, 100, 0, 100, False),
])
def test_dense_formulation(cfg):
    rows, qh, kvh, d, p, t, b, e, int8 = cfg
    case = W.synth_case(rows, qh, kvh, d, p, t, seed=sum(cfg[:8]), begin=b, end=e,
                        qpos=np.linspace(b, t, rows).astype(np.int64), int8=int8)
    got, gvis = O.fp64(case)
    ref, rvis = dense_fp64(case)
    assert np.array_equal(gvis, rvis)
    assert np.max(np.abs(got - ref), initial=0.0) <= 1e-10


# ---- split + merge (fp32) ----------------------------------------------------

def split_merge_ok(case, split_tokens, tol=2e-5):
    sc, splits = O.split_fp32(case, split_tokens, threads=4)
    m, l, n = O.merge_fp32(case.shape, sc, splits)
    out, vis, ok = O.normalize(m, l, n, case.shape.dim)
    ref, rvis = O.fp64(case, threads=4)
    if not ok or not np.array_equal(vis, rvis):
        return False
    return bool(np.all(np.abs(out - ref) <= tol * max(1.0, np.abs(ref).max(initial=0.0))))


def split_cases():
    yield W.synth_case(2, 8, 2, 64, 16, 700, seed=5, begin=33, end=650, qpos=[300, 700])
    c = W.synth_case(1, 4, 2, 32, 32, 300, seed=6, begin=40, end=300)
    c.qpos = np.array([-1], np.int64)  # every split empty
    yield c


@pytest.mark.parametrize("split_tokens", [1, 7, 64, 256, 1000])
def test_split_merge_matches_fp64(split_tokens):
    for case in split_cases():
        assert split_merge_ok(case, split_tokens)


def test_single_split_merge_is_identity():
    case = W.synth_case(1, 8, 2, 64, 16, 300, seed=8)
    sc, splits = O.split_fp32(case, 4096)
    assert splits == 1
    m, l, n = O.merge_fp32(case.shape, sc, splits)
    part = sc.reshape(8, 66)
    assert np.array_equal(m, part[:, 0]) and np.array_equal(l, part[:, 1])
    assert np.array_equal(n.reshape(8, 64), part[:, 2:])


def test_all_empty_convention():
    case = W.synth_case(1, 4, 2, 32, 16, 100, seed=9, qpos=[-5])
    sc, splits = O.split_fp32(case, 16)
    m, l, n = O.merge_fp32(case.shape, sc, splits)
    assert np.all(np.isneginf(m)) and np.all(l == 0) and np.all(n == 0)


# ---- planted mistakes --------------------------------------------------------

def check_battery():
    """Every check above as a (name, passed) list, for the planted-fault test."""
    results = [
        ("zero_q_closed_form", zero_q_closed_form_ok()),
        ("permutation_invariance", permutation_invariant_ok()),
        ("future_poison", future_poison_ok()),
        ("empty_and_masked", empty_and_masked_ok()),
    ]
    results += [(f"golden:{os.path.basename(p)}", golden_ok(p)) for p in GOLDEN]
    results += [(f"split_merge:{st}", all(split_merge_ok(c, st) for c in split_cases())) for st in (7, 256)]
    return results


def test_battery_passes_on_faithful_oracle():
    failed = [n for n, ok in check_battery() if not ok]
    assert not failed, failed


ATTENTION_FAULTS = sorted(f for f in O.FAULTS if not f.startswith("quant_"))  # quant_*: test_append_oracle.py


@pytest.mark.parametrize("fault", ATTENTION_FAULTS, ids=ATTENTION_FAULTS)
def test_planted_fault_is_caught(fault):
    O.set_fault(O.FAULTS[fault])
    try:
        caught = [n for n, ok in check_battery() if not ok]
    finally:
        O.set_fault(0)
    assert caught, f"planted fault {fault} passed every check"
