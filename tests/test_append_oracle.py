"""CPU checks of the quantizing append restatement (oracle_append_int8):
known answers (ties round to even, all-zero rows get scale 1, +-absmax maps
to +-127), an independent numpy formulation (the synthetic-data quantizer,
scattered into the page layout) on random and tie-heavy rows, padding slots,
and planted mistakes that these checks must catch."""
import numpy as np
import pytest

from kvbridge_amd import workloads as W
from oracle import oracle as O


def empty_pool(pages, kvh, P, D):
    rng = np.random.default_rng(0)
    k = rng.integers(-128, 128, (pages, kvh, P, D), dtype=np.int8)
    v = rng.integers(-128, 128, (pages, kvh, D, P), dtype=np.int8)
    ks = rng.random((pages, kvh, P), dtype=np.float32)
    vs = rng.random((pages, kvh, P), dtype=np.float32)
    return k, v, ks, vs


def numpy_append(pool, kn, vn, slots, P):
    """Independent formulation: quantize_rows per (token, kv head), then scatter."""
    k, v, ks, vs = (np.array(a, copy=True) for a in pool)
    kc, kscale = W.quantize_rows(kn)
    vc, vscale = W.quantize_rows(vn)
    pages = k.shape[0]
    for t, sid in enumerate(slots):
        if sid >= pages * P:
            continue
        page, slot = divmod(int(sid), P)
        k[page, :, slot, :] = kc[t]
        v[page, :, :, slot] = vc[t]
        ks[page, :, slot] = kscale[t]
        vs[page, :, slot] = vscale[t]
    return k, v, ks, vs


def test_known_answers():
    pool = empty_pool(2, 1, 4, 3)
    kn = np.array([[[127., 0.5, -1.5]], [[0, 0, 0]]], np.float32)
    vn = np.array([[[2.5, -2.5, 127]], [[1, 2, 3]]], np.float32)
    k, v, ks, vs = O.append_int8(*pool, kn, vn, np.array([5, 1], np.uint32), 4)
    assert k[1, 0, 1].tolist() == [127, 0, -2] and ks[1, 0, 1] == 1.0
    assert v[1, 0, :, 1].tolist() == [2, -2, 127] and vs[1, 0, 1] == 1.0
    assert k[0, 0, 1].tolist() == [0, 0, 0] and ks[0, 0, 1] == 1.0
    assert v[0, 0, :, 1].tolist() == [42, 85, 127] and vs[0, 0, 1] == np.float32(3) / np.float32(127)
    # untouched slots keep their contents
    assert np.array_equal(k[0, 0, 0], pool[0][0, 0, 0]) and v[0, 0, 0, 0] == pool[1][0, 0, 0, 0]


@pytest.mark.parametrize("D,kvh,P,tokens", [(128, 8, 64, 200), (64, 2, 16, 97), (67, 3, 32, 50), (256, 1, 64, 33)])
def test_matches_numpy_formulation(D, kvh, P, tokens):
    rng = np.random.default_rng(D * 1000 + tokens)
    pages = -(-tokens // P) + 2
    pool = empty_pool(pages, kvh, P, D)
    kn = rng.standard_normal((tokens, kvh, D), dtype=np.float32)
    vn = rng.standard_normal((tokens, kvh, D), dtype=np.float32) * 3
    kn[0, 0] = 0.0                                    # all-zero row
    vn[1, :, :] = np.round(vn[1] * 2) / 2             # many exact halves after scaling by 1
    vn[1, :, 0] = 127.0                               # absmax 127 -> scale exactly 1 -> ties at .5
    slots = rng.permutation(pages * P)[:tokens].astype(np.uint32)
    slots[3] = 0xFFFFFFFF                             # padding entry: skipped
    got = O.append_int8(*pool, kn, vn, slots, P)
    want = numpy_append(pool, kn, vn, slots, P)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("fault", ["quant_round_away", "quant_scale_128", "quant_v_token_major"])
def test_planted_mistakes_are_caught(fault):
    rng = np.random.default_rng(5)
    P, D, kvh, tokens = 16, 64, 2, 40
    pool = empty_pool(4, kvh, P, D)
    kn = rng.standard_normal((tokens, kvh, D), dtype=np.float32)
    vn = np.round(rng.standard_normal((tokens, kvh, D), dtype=np.float32) * 8) / 2
    vn[:, :, 0] = 127.0
    slots = rng.permutation(4 * P)[:tokens].astype(np.uint32)
    want = numpy_append(pool, kn, vn, slots, P)
    O.set_fault(O.FAULTS[fault])
    try:
        got = O.append_int8(*pool, kn, vn, slots, P)
    finally:
        O.set_fault(0)
    assert not all(np.array_equal(g, w) for g, w in zip(got, want)), fault


def numpy_quantize_nonfinite(x):
    """Independent formulation of the rule for any fp32 rows: absmax by
    np.fmax (NaN left out), scale = absmax / 127 (1 for 0), code =
    fmin(fmax(rint(x / scale), -127), 127) with fmax / fmin NaN-ignoring, so a
    NaN quotient gives -127."""
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        absmax = np.fmax.reduce(np.abs(x), axis=-1, initial=np.float32(0)).astype(np.float32)
        scale = np.where(absmax == 0, np.float32(1), (absmax / np.float32(127)).astype(np.float32))
        q = (x / scale[..., None]).astype(np.float32)
        code = np.fmin(np.fmax(np.rint(q), np.float32(-127)), np.float32(127)).astype(np.int8)
    return code, scale


def test_non_finite_known_answers():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    pool = empty_pool(1, 1, 4, 4)
    kn = np.array([[[nan, 1.0, -2.0, 0.5]],     # NaN left out of the absmax: scale 2/127, NaN -> -127
                   [[inf, 1.0, -3.0, -inf]],    # infinite scale: finite -> 0, +-inf (inf/inf = NaN) -> -127
                   [[nan, nan, nan, nan]]],     # absmax 0: scale 1, every code -127
                  np.float32)
    vn = np.zeros_like(kn)
    k, v, ks, vs = O.append_int8(*pool, kn, vn, np.array([0, 1, 2], np.uint32), 4)
    assert k[0, 0, 0].tolist() == [-127, 64, -127, 32] and ks[0, 0, 0] == np.float32(2) / np.float32(127)
    assert k[0, 0, 1].tolist() == [-127, 0, 0, -127] and np.isposinf(ks[0, 0, 1])
    assert k[0, 0, 2].tolist() == [-127] * 4 and ks[0, 0, 2] == 1.0
    assert vs[0, 0, :3].tolist() == [1.0, 1.0, 1.0]


def test_non_finite_matches_numpy_formulation():
    rng = np.random.default_rng(11)
    tokens, kvh, D, P = 64, 2, 96, 16
    pool = empty_pool(5, kvh, P, D)
    kn = rng.standard_normal((tokens, kvh, D), dtype=np.float32)
    vn = rng.standard_normal((tokens, kvh, D), dtype=np.float32)
    for a in (kn, vn):
        hit = rng.random(a.shape) < 0.02
        a[hit] = rng.choice(np.array([np.nan, np.inf, -np.inf], np.float32), hit.sum())
    kn[5, 1] = np.nan
    vn[7, 0, :] = np.inf
    slots = rng.permutation(5 * P)[:tokens].astype(np.uint32)
    k, v, ks, vs = O.append_int8(*pool, kn, vn, slots, P)
    kc, kscale = numpy_quantize_nonfinite(kn)
    vc, vscale = numpy_quantize_nonfinite(vn)
    for t, sid in enumerate(slots):
        page, slot = divmod(int(sid), P)
        assert np.array_equal(k[page, :, slot, :], kc[t]) and np.array_equal(v[page, :, :, slot], vc[t])
        assert np.array_equal(ks[page, :, slot].view(np.uint32), kscale[t].view(np.uint32))
        assert np.array_equal(vs[page, :, slot].view(np.uint32), vscale[t].view(np.uint32))


def test_fast_scale_division_is_the_ieee_quotient():
    """The append kernels compute absmax / 127 as q0 = RN(a * RN(1/127)) plus
    one fma residual step (append.hip scale_of).  tests/cpp/scale_div_check.c
    compares it bitwise with IEEE single division on every 61st non-negative
    finite fp32 bit pattern and on every value an fp16 row maximum can take
    (its full sweep, stride 1, also finds no mismatch).  A planted mistake --
    the first product alone, without the residual step -- must be caught."""
    import subprocess
    from pathlib import Path
    here = Path(__file__).resolve().parent / "cpp"
    subprocess.run(["make", "-s", "-C", str(here), "scale_div_check"], check=True)
    r = subprocess.run([str(here / "scale_div_check")], capture_output=True, text=True)
    assert r.returncode == 0 and " 0 mismatches" in r.stdout, r.stdout
    # the planted mistake, restated in numpy: RN(a * RN(1/127)) without the correction
    rng = np.random.default_rng(5)
    a = rng.uniform(0, 1e4, 200_000).astype(np.float32)
    c = np.float32(1) / np.float32(127)
    assert np.any((a * c) != (a / np.float32(127)))


def test_fma_quotient_is_the_ieee_quotient_for_16_bit_sources():
    """For fp16 and bf16 sources the row-streaming append kernel takes the
    quotient x / scale as q0 = RN(x * r), q = fma(fma(-q0, scale, x), r, q0)
    with r the hardware reciprocal (append.hip quantize_lane), with no check.
    tests/cpp/quant_fmadiv_check.c compares rint(q) with rint of the IEEE
    quotient for every 3rd fp16 / 5th bf16 row maximum, every fp32 r within
    one ulp of 1/scale and every source value below the maximum, both signs
    (its stride-1 sweeps, 2.0e9 fp16 and 2.1e9 bf16 cases, also find no
    mismatch).  Planted mistakes -- q0 without the residual step, and bf16
    rows below the kernel's 2^-100 scale cutoff -- must be caught."""
    import subprocess
    from pathlib import Path
    here = Path(__file__).resolve().parent / "cpp"
    subprocess.run(["make", "-s", "-C", str(here), "quant_fmadiv_check"], check=True)
    exe = str(here / "quant_fmadiv_check")
    for fmt, stride in (("fp16", "3"), ("bf16", "5")):
        r = subprocess.run([exe, fmt, stride], capture_output=True, text=True)
        assert r.returncode == 0 and " 0 mismatches" in r.stdout, r.stdout
    for fmt, mode in (("fp16", "1"), ("bf16", "2")):
        bad = subprocess.run([exe, fmt, "3", mode], capture_output=True, text=True)
        assert bad.returncode == 1 and " 0 mismatches" not in bad.stdout, (fmt, mode, bad.stdout)


def test_bracketed_code_rounding_is_the_ieee_quotient():
    """The row-streaming append kernel rounds x / scale to its code (fp32
    sources) from two
    fmas, x * RN(r * (1 -+ 2^-21)) + 1.5 * 2^23 with r the hardware
    reciprocal, and divides only where the two disagree (append.hip
    quantize_lane).  tests/cpp/quant_bracket_check.c checks that agreement
    implies rint(RN(x / scale)) for every fp32 r within one ulp of 1/scale,
    every 5th fp16 row maximum with every fp16 source value below it (both
    signs), and random fp32 rows including their exact ties (its full fp16
    sweep, stride 1, also finds no mismatch).  Planted mistakes -- a bracket of
    2^-23, too narrow for the reciprocal's ulp, and no bracket at all -- must
    be caught."""
    import subprocess
    from pathlib import Path
    here = Path(__file__).resolve().parent / "cpp"
    subprocess.run(["make", "-s", "-C", str(here), "quant_bracket_check"], check=True)
    exe = str(here / "quant_bracket_check")
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0 and " 0 mismatches" in r.stdout, r.stdout
    for k in ("23", "0"):
        bad = subprocess.run([exe, "37", "200000", k], capture_output=True, text=True)
        assert bad.returncode == 1 and " 0 mismatches" not in bad.stdout, (k, bad.stdout)
