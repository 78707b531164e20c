"""TEST INFRASTRUCTURE ONLY: ctypes front of the CPU oracle (liboracle.so) and
of the reference's own FP64 oracle built from source (_ref/libkvbridge_ref.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker or the timed CPU baseline.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libkvbridge_ref.so")


class OShape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("rows", "q_heads", "kv_heads", "dim", "page_tokens", "pages", "tokens", "begin", "end")] + \
               [("scale", ctypes.c_float), ("int8", ctypes.c_uint32)]


def _oshape(s) -> OShape:
    return OShape(s.rows, s.q_heads, s.kv_heads, s.dim, s.page_tokens, s.pages, s.tokens, s.begin, s.end,
                  s.scale, s.int8)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(ORACLE_SO)
    return _lib


# Planted mistakes (attention_oracle.h ORACLE_FAULT_*), for the tests that
# show the oracle's checks catch them.
FAULTS = {
    "kscale_dropped": 1,
    "vscale_dropped": 2,
    "scale_dropped": 3,
    "mask_strict": 4,
    "table_ignored": 5,
    "v_token_major": 6,
    "gqa_modulo": 7,
    "split_ignores_begin": 8,
    "merge_no_skip": 9,
    "quant_round_away": 10,
    "quant_scale_128": 11,
    "quant_v_token_major": 12,
}


def set_fault(code: int) -> None:
    lib().oracle_set_fault(ctypes.c_int(code))


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        _ref = ctypes.CDLL(REF_SO)
    return _ref


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _arrays(case):
    c = case
    return [np.ascontiguousarray(x) for x in (c.q, c.qpos, c.kpos, c.table, c.k, c.v, c.ks, c.vs)]


def fp64(case, threads: int = 1):
    """FP64 normalized output [rows*q_heads, dim] and visibility [rows*q_heads]."""
    s = case.shape
    arrs = _arrays(case)
    out = np.zeros((s.rows * s.q_heads, s.dim), np.float64)
    vis = np.zeros(s.rows * s.q_heads, np.uint8)
    sh = _oshape(s)
    lib().oracle_fp64(ctypes.byref(sh), *[_p(a) for a in arrs], _p(out), _p(vis), ctypes.c_int(threads))
    return out, vis.astype(bool)


def split_fp32(case, split_tokens: int, threads: int = 1):
    s = case.shape
    length = s.end - s.begin
    splits = max(1, -(-length // split_tokens))
    scratch = np.zeros(s.rows * s.q_heads * splits * (s.dim + 2), np.float32)
    arrs = _arrays(case)
    sh = _oshape(s)
    lib().oracle_split_fp32(ctypes.byref(sh), *[_p(a) for a in arrs], ctypes.c_uint32(split_tokens),
                            ctypes.c_uint32(splits), _p(scratch), ctypes.c_int(threads))
    return scratch, splits


def merge_fp32(shape, scratch: np.ndarray, splits: int):
    rh = shape.rows * shape.q_heads
    m = np.zeros(rh, np.float32)
    l = np.zeros(rh, np.float32)
    n = np.zeros(rh * shape.dim, np.float32)
    sc = np.ascontiguousarray(scratch, np.float32)
    sh = _oshape(shape)
    lib().oracle_merge_fp32(ctypes.byref(sh), _p(sc), ctypes.c_uint32(splits), _p(m), _p(l), _p(n))
    return m, l, n


def fixture(tokens: int, permute: bool = False):
    """The reference's closed-form fixture (attention_reference.h:19-48) as a Case."""
    from kvbridge_amd.workloads import Case
    from kvbridge_amd._capi import Shape

    P, kv, D, rows, qh = 32, 4, 256, 8, 24
    pages = -(-tokens // P)
    q = np.zeros(rows * qh * D, np.float32)
    qpos = np.zeros(rows, np.int64)
    kpos = np.zeros(tokens, np.int64)
    table = np.zeros(pages, np.uint32)
    k = np.zeros((pages, kv, P, D), np.int8)
    v = np.zeros((pages, kv, D, P), np.int8)
    ks = np.zeros((pages, kv, P), np.float32)
    vs = np.zeros((pages, kv, P), np.float32)
    lib().oracle_fixture(ctypes.c_uint32(tokens), ctypes.c_int(1 if permute else 0), _p(q), _p(qpos), _p(kpos),
                         _p(table), _p(k), _p(v), _p(ks), _p(vs))
    shape = Shape(rows, qh, kv, D, P, pages, tokens, 0, tokens, 0.0625, 1)
    return Case(shape, q, qpos, kpos, table, k, v, ks, vs, meta={"fixture": tokens, "permute": permute})


def ref_fp64(case):
    """The reference's own FP64 oracle (INT8 KV only), built from its sources."""
    s = case.shape
    arrs = _arrays(case)
    out = np.zeros((s.rows * s.q_heads, s.dim), np.float64)
    vis = np.zeros(s.rows * s.q_heads, np.uint8)
    sh = _oshape(s)
    rc = ref().ref_fp64_oracle(ctypes.byref(sh), *[_p(a) for a in arrs], _p(out), _p(vis))
    if rc != 0:
        raise ValueError("reference oracle rejected the shape")
    return out, vis.astype(bool)


def ref_fixture(tokens: int, permute: bool = False):
    """The reference's make_fixture output, for pinning oracle_fixture."""
    base = fixture(tokens, permute)
    arrs = [np.zeros_like(x) for x in (base.q, base.qpos, base.kpos, base.table, base.k, base.v, base.ks, base.vs)]
    ref().ref_make_fixture(ctypes.c_uint(tokens), ctypes.c_int(1 if permute else 0), *[_p(a) for a in arrs])
    return arrs


def normalize(m, l, n, dim):
    """Caller normalization of the reference harness (examples/attention_bench.cu:98-116):
    out = n / l where l > 0; l == 0 rows must have m = -inf and n = 0 and give zeros.
    Returns (out float64 [rh, dim], visible bool [rh], ok)."""
    m = np.asarray(m, np.float64)
    l = np.asarray(l, np.float64)
    n = np.asarray(n, np.float64).reshape(-1, dim)
    vis = l > 0
    ok = True
    empty = ~vis
    if np.any(empty):
        ok &= bool(np.all(np.isneginf(m[empty]))) and bool(np.all(n[empty] == 0))
    ok &= bool(np.all(np.isfinite(l))) and bool(np.all(l >= 0))
    ok &= bool(np.all(np.isfinite(m[vis]))) and bool(np.all(np.isfinite(n[vis])))
    out = np.zeros_like(n)
    out[vis] = n[vis] / l[vis, None]
    return out, vis, ok


def gates(actual: np.ndarray, ref: np.ndarray):
    """North-star gate (max-abs <= 2e-3 and relative L2 <= 1e-3) plus the
    reference's stricter per-element oracle gate |a - r| <= 3e-6 + 5e-5|r|
    (examples/attention_bench.cu:127), reported separately."""
    a = np.asarray(actual, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    err = np.abs(a - r)
    max_abs = float(err.max()) if err.size else 0.0
    denom = float(np.linalg.norm(r))
    rel_l2 = float(np.linalg.norm(a - r) / denom) if denom > 0 else float(np.linalg.norm(a - r))
    strict = bool(np.all(err <= 3e-6 + 5e-5 * np.abs(r)))
    return {"max_abs": max_abs, "rel_l2": rel_l2, "pass": max_abs <= 2e-3 and rel_l2 <= 1e-3, "strict_pass": strict}


def append_int8(pool_k, pool_v, pool_ks, pool_vs, k_new, v_new, slots, page_tokens):
    """Quantizing append into copies of the pool arrays (oracle_append_int8).
    pool_k int8 [pages, kv, P, D], pool_v int8 [pages, kv, D, P], scales [pages, kv, P];
    k_new / v_new float32 [tokens, kv, D]; slots uint32 [tokens]."""
    k, v = np.array(pool_k, np.int8, copy=True), np.array(pool_v, np.int8, copy=True)
    ks, vs = np.array(pool_ks, np.float32, copy=True), np.array(pool_vs, np.float32, copy=True)
    kn = np.ascontiguousarray(k_new, np.float32)
    vn = np.ascontiguousarray(v_new, np.float32)
    sl = np.ascontiguousarray(slots, np.uint32)
    tokens, kvh, dim = kn.shape
    pages = k.shape[0]
    lib().oracle_append_int8(ctypes.c_uint32(tokens), ctypes.c_uint32(kvh), ctypes.c_uint32(dim),
                             ctypes.c_uint32(page_tokens), ctypes.c_uint32(pages), _p(kn), _p(vn),
                             ctypes.c_uint32(kvh * dim), ctypes.c_uint32(kvh * dim), _p(sl), _p(k), _p(v), _p(ks),
                             _p(vs))
    return k, v, ks, vs
