"""Paged INT8 KV append (kvb_append_kv) on the GPU: codes and scales are
bitwise those of the CPU restatement (oracle_append_int8) for fp32, fp16 and
bf16 sources, strided sources, padding slots and odd head dims, untouched
slots keep their bytes; and a cache written token by token through the
append path is bitwise the cache the synthetic generator builds, and decodes
to the FP64 oracle's output."""
import numpy as np
import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import DeviceCase, check_against_oracle, log

pytestmark = pytest.mark.gpu

SRC = {kvb.KVB_SRC_F32: "float32", kvb.KVB_SRC_F16: "float16", kvb.KVB_SRC_BF16: "bfloat16"}


def random_pool(pages, kvh, P, D, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(-128, 128, (pages, kvh, P, D), dtype=np.int8),
            rng.integers(-128, 128, (pages, kvh, D, P), dtype=np.int8),
            rng.random((pages, kvh, P), dtype=np.float32), rng.random((pages, kvh, P), dtype=np.float32))


CASES = [
    # tokens, kv_heads, dim, page, src, extra stride (elements)
    (300, 8, 128, 64, kvb.KVB_SRC_F32, 0),
    (77, 8, 128, 64, kvb.KVB_SRC_F16, 0),
    (129, 2, 64, 16, kvb.KVB_SRC_BF16, 0),
    (50, 3, 67, 32, kvb.KVB_SRC_F32, 0),
    (40, 1, 256, 64, kvb.KVB_SRC_F16, 0),
    (64, 8, 128, 64, kvb.KVB_SRC_BF16, 4096),   # rows inside a wider (fused QKV-like) buffer
    (1, 8, 128, 64, kvb.KVB_SRC_F32, 0),        # one decode-step token
    # >= 256 tokens: the tile kernel (lane = token)
    (300, 8, 128, 64, kvb.KVB_SRC_F16, 0),       # 16-byte loads and K stores
    (400, 3, 67, 32, kvb.KVB_SRC_F32, 0),        # odd dim: element path
    (260, 1, 256, 64, kvb.KVB_SRC_BF16, 0),
    (512, 8, 128, 64, kvb.KVB_SRC_BF16, 4096),   # rows inside a wider buffer
    (257, 2, 100, 16, kvb.KVB_SRC_F16, 3),       # stride not a 16-byte multiple: element path
    (288, 2, 256, 64, kvb.KVB_SRC_F16, 0),       # row-streaming, dim 256, random slots
    (320, 2, 128, 48, kvb.KVB_SRC_F32, 0),       # row-streaming, page size not a power of two
]


def _run_append(gpu, tokens, kvh, D, P, src, extra, slots, pages, seed):
    import torch

    rng = np.random.default_rng(seed)
    pool = random_pool(pages, kvh, P, D, seed=tokens)
    row = kvh * D
    stride = row + extra
    tdt = getattr(torch, SRC[src])
    kbuf = torch.from_numpy(rng.standard_normal((tokens, stride), dtype=np.float32) * 2).to(tdt)
    vbuf = torch.from_numpy(rng.standard_normal((tokens, stride), dtype=np.float32) * 0.5).to(tdt)
    kbuf[0, :D] = 0                                   # an all-zero row
    vbuf[-1, :D] = torch.tensor(np.round(rng.standard_normal(D) * 4) / 2, dtype=tdt)  # exact halves
    vbuf[-1, 0] = 127
    # host reference on the exactly representable fp32 values of the source
    kn = kbuf.float().numpy()[:, :row].reshape(tokens, kvh, D)
    vn = vbuf.float().numpy()[:, :row].reshape(tokens, kvh, D)
    want = O.append_int8(*pool, kn, vn, slots, P)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in pool]
    s = kvb.append_shape(tokens, kvh, D, P, pages, src, stride, stride)
    log(f"append tokens={tokens} kv={kvh} dim={D} page={P} src={SRC[src]} stride={stride}")
    kvb.append_kv(s, kbuf.to(gpu), vbuf.to(gpu), torch.from_numpy(slots.view(np.int32)).to(gpu), *dev)
    torch.cuda.synchronize()
    for name, g, w in zip(("k", "v", "k_scales", "v_scales"), dev, want):
        got = g.cpu().numpy()
        assert np.array_equal(got.view(np.uint8) if got.dtype == np.int8 else got.view(np.uint32),
                              w.view(np.uint8) if w.dtype == np.int8 else w.view(np.uint32)), f"{name} differs"


@pytest.mark.parametrize("case", CASES)
def test_append_matches_oracle_bitwise(gpu, case):
    tokens, kvh, D, P, src, extra = case
    rng = np.random.default_rng(tokens * 31 + D)
    pages = -(-tokens // P) + 3
    slots = rng.permutation(pages * P)[:tokens].astype(np.uint32)
    if tokens > 3:
        slots[2] = 0xFFFFFFFF                         # padding entry
    _run_append(gpu, tokens, kvh, D, P, src, extra, slots, pages, seed=tokens * 31 + D)


PREFILL_CASES = [
    # tokens, kv_heads, dim, page, src, first slot offset in its page, padding entries
    (4096, 8, 128, 64, kvb.KVB_SRC_F16, 0, ()),       # whole pages: every 16-slot group is one V store
    (1000, 2, 256, 32, kvb.KVB_SRC_F32, 0, ()),       # ragged last tile and group
    (700, 4, 64, 16, kvb.KVB_SRC_BF16, 8, ()),        # groups straddle 16-slot boundaries: byte stores
    (520, 8, 128, 64, kvb.KVB_SRC_F16, 0, (100, 263)),  # padding inside two groups
    (300, 1, 64, 64, kvb.KVB_SRC_F32, 48, ()),        # starts mid-page, crosses pages
    (600, 2, 256, 48, kvb.KVB_SRC_F16, 0, ()),        # page size not a power of two (division path)
    (400, 3, 128, 80, kvb.KVB_SRC_BF16, 16, (5,)),    # same, mid-page start, a padding entry
]


@pytest.mark.parametrize("case", PREFILL_CASES)
def test_append_prefill_mapping_matches_oracle_bitwise(gpu, case):
    """A prefill chunk's slot mapping (consecutive slots of permuted pages),
    the layout the row-streaming kernel stores 16 V codes at a time."""
    tokens, kvh, D, P, src, off, pads = case
    rng = np.random.default_rng(tokens * 7 + D)
    pages = -(-(tokens + off) // P) + 2
    order = rng.permutation(pages).astype(np.uint32)
    t = np.arange(tokens, dtype=np.uint32) + off
    slots = (order[t // P] * P + t % P).astype(np.uint32)
    for i in pads:
        slots[i] = 0xFFFFFFFF
    _run_append(gpu, tokens, kvh, D, P, src, 0, slots, pages, seed=tokens * 7 + D)


NEAR_TIE_CASES = [
    # tokens, kv_heads, dim, page, src: the row, tile and row-streaming kernels
    (3, 4, 128, 64, kvb.KVB_SRC_F32),
    (300, 4, 67, 32, kvb.KVB_SRC_F32),
    (320, 4, 128, 64, kvb.KVB_SRC_F32),
    (320, 4, 128, 64, kvb.KVB_SRC_F16),
    (320, 4, 128, 64, kvb.KVB_SRC_BF16),
    (320, 2, 64, 16, kvb.KVB_SRC_F16),
    (288, 2, 256, 32, kvb.KVB_SRC_F32),
]


@pytest.mark.parametrize("case", NEAR_TIE_CASES)
def test_append_near_ties_matches_oracle_bitwise(gpu, case):
    """Elements whose quotient x / scale lies within a few ulp of a
    half-integer (or exactly on one), where the kernels' reciprocal fast path
    must defer to the correctly rounded division: codes bitwise the CPU
    quantizer's (rint of the fp32 quotient, ties to even)."""
    import torch

    tokens, kvh, D, P, src = case
    rng = np.random.default_rng(tokens * 13 + D + src)
    pages = -(-tokens // P) + 1
    slots = rng.permutation(pages * P)[:tokens].astype(np.uint32)
    tdt = getattr(torch, SRC[src])
    bufs = []
    for _ in range(2):
        amax = (rng.random((tokens, kvh, 1)) * 4 + 0.25).astype(np.float32)
        amax = torch.from_numpy(amax).to(tdt).float().numpy()     # representable in the source type
        scale = (amax / np.float32(127)).astype(np.float32)
        k = rng.integers(-127, 127, (tokens, kvh, D)).astype(np.float32) + np.float32(0.5)
        x = (k * scale).astype(np.float32)                         # at or next to a tie
        steps = rng.integers(-3, 4, (tokens, kvh, D))
        for _s in range(3):                                        # move up to 3 ulp either way
            x = np.where(steps > _s, np.nextafter(x, np.float32(np.inf)), x)
            x = np.where(-steps > _s, np.nextafter(x, np.float32(-np.inf)), x)
        x = np.clip(x, -amax, amax)
        x[..., 0] = amax[..., 0]                                   # the row's absmax itself
        xt = torch.from_numpy(x.astype(np.float32)).to(tdt)        # fp16 sources round to near-ties of their own
        bufs.append(xt.reshape(tokens, kvh * D))
    kbuf, vbuf = bufs
    pool = random_pool(pages, kvh, P, D, seed=tokens)
    kn = kbuf.float().numpy().reshape(tokens, kvh, D)
    vn = vbuf.float().numpy().reshape(tokens, kvh, D)
    want = O.append_int8(*pool, kn, vn, slots, P)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in pool]
    s = kvb.append_shape(tokens, kvh, D, P, pages, src)
    log(f"near-tie append tokens={tokens} kv={kvh} dim={D} page={P} src={SRC[src]}")
    kvb.append_kv(s, kbuf.to(gpu), vbuf.to(gpu), torch.from_numpy(slots.view(np.int32)).to(gpu), *dev)
    torch.cuda.synchronize()
    for name, g, w in zip(("k", "v", "k_scales", "v_scales"), dev, want):
        got = g.cpu().numpy()
        assert np.array_equal(got.view(np.uint8) if got.dtype == np.int8 else got.view(np.uint32),
                              w.view(np.uint8) if w.dtype == np.int8 else w.view(np.uint32)), f"{name} differs"


NON_FINITE_CASES = [
    # tokens, kv_heads, dim, page, src: the row, tile and row-streaming kernels
    (5, 4, 128, 64, kvb.KVB_SRC_F32),
    (5, 4, 128, 64, kvb.KVB_SRC_F16),
    (300, 3, 67, 32, kvb.KVB_SRC_F32),
    (300, 3, 67, 32, kvb.KVB_SRC_F16),
    (320, 4, 128, 64, kvb.KVB_SRC_F32),
    (320, 4, 128, 64, kvb.KVB_SRC_F16),
    (320, 4, 128, 64, kvb.KVB_SRC_BF16),
]


@pytest.mark.parametrize("case", NON_FINITE_CASES)
def test_append_non_finite_sources_match_oracle_bitwise(gpu, case):
    """Rows holding NaN and +-infinity: every kernel follows the one rule of
    the oracle (NaN left out of the absmax, an infinite element makes the
    scale infinite, a NaN quotient clamps to -127), bitwise.  Rows of tiny
    magnitudes (fp32 and bf16 sources) have scales below 2^-100, one of them
    below the normal range, where the row-streaming kernel divides."""
    import torch

    tokens, kvh, D, P, src = case
    rng = np.random.default_rng(tokens * 17 + D + src)
    pages = -(-tokens // P) + 1
    slots = rng.permutation(pages * P)[:tokens].astype(np.uint32)
    tdt = getattr(torch, SRC[src])
    bufs = []
    for _ in range(2):
        x = rng.standard_normal((tokens, kvh, D), dtype=np.float32) * 2
        hit = rng.random(x.shape) < 0.01
        x[hit] = rng.choice(np.array([np.nan, np.inf, -np.inf], np.float32), hit.sum())
        x[1, 0, 3] = np.nan                        # a NaN in an otherwise finite row
        x[2, 0, 5] = np.inf                        # an infinite element: infinite scale
        x[3, 0, :] = np.nan                        # an all-NaN row: scale 1, codes -127
        x[4, 0, :] = rng.standard_normal(D, dtype=np.float32) * np.float32(1e-39)  # subnormal scale
        if tokens > 6:
            x[5, 0, :] = rng.standard_normal(D, dtype=np.float32) * np.float32(1e-33)  # scale ~2^-115
            x[6, 0, :] = rng.standard_normal(D, dtype=np.float32) * np.float32(1e-36)  # scale near 2^-125
        bufs.append(torch.from_numpy(x.reshape(tokens, kvh * D)).to(tdt))
    kbuf, vbuf = bufs
    pool = random_pool(pages, kvh, P, D, seed=tokens)
    kn = kbuf.float().numpy().reshape(tokens, kvh, D)
    vn = vbuf.float().numpy().reshape(tokens, kvh, D)
    want = O.append_int8(*pool, kn, vn, slots, P)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in pool]
    s = kvb.append_shape(tokens, kvh, D, P, pages, src)
    log(f"non-finite append tokens={tokens} kv={kvh} dim={D} page={P} src={SRC[src]}")
    kvb.append_kv(s, kbuf.to(gpu), vbuf.to(gpu), torch.from_numpy(slots.view(np.int32)).to(gpu), *dev)
    torch.cuda.synchronize()
    for name, g, w in zip(("k", "v", "k_scales", "v_scales"), dev, want):
        got = g.cpu().numpy()
        assert np.array_equal(got.view(np.uint8) if got.dtype == np.int8 else got.view(np.uint32),
                              w.view(np.uint8) if w.dtype == np.int8 else w.view(np.uint32)), f"{name} differs"


@pytest.mark.parametrize("src", [kvb.KVB_SRC_F16, kvb.KVB_SRC_BF16])
def test_append_every_16_bit_row_maximum_matches_oracle_bitwise(gpu, src):
    """Every positive finite fp16 (bf16) value as a row maximum, through the
    row-streaming kernel, whose fp16 / bf16 codes come from an fma quotient
    with the hardware reciprocal and no check (exact for every reciprocal
    within one ulp: tests/cpp/quant_fmadiv_check.c): one token per maximum,
    its other elements the maximum times (2j + 1) / 254 (quotients at or next
    to the half-integers) and random fractions of it with either sign, codes
    and scales bitwise the CPU quantizer's.  bf16 maxima reach scales below
    2^-100, which divide."""
    import torch

    if src == kvb.KVB_SRC_F16:
        vals = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    else:
        vals = (np.arange(1, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    tokens, kvh, D, P = len(vals), 1, 128, 64
    rng = np.random.default_rng(0x7C00 + src)
    x = np.empty((tokens, D), np.float64)
    x[:, 0] = vals
    x[:, 1:64] = vals[:, None].astype(np.float64) * (2 * np.arange(63) + 1) / 254.0
    x[:, 64:] = vals[:, None].astype(np.float64) * rng.uniform(-1, 1, (tokens, 64))
    tdt = getattr(torch, SRC[src])
    bufs = []
    for sgn in (1.0, -1.0):                     # K rows as built, V rows negated
        t = torch.from_numpy((sgn * x).astype(np.float32)).to(tdt)
        assert torch.equal(t[:, 0].float().abs(), torch.from_numpy(vals))  # the maxima are exact
        bufs.append(t)
    kbuf, vbuf = bufs
    assert (kbuf.float().abs().max(dim=1).values == kbuf[:, 0].float().abs()).all()
    pages = -(-tokens // P) + 1
    order = rng.permutation(pages).astype(np.uint32)
    tk = np.arange(tokens, dtype=np.uint32)
    slots = (order[tk // P] * P + tk % P).astype(np.uint32)
    pool = random_pool(pages, kvh, P, D, seed=11)
    kn = kbuf.float().numpy().reshape(tokens, kvh, D)
    vn = vbuf.float().numpy().reshape(tokens, kvh, D)
    want = O.append_int8(*pool, kn, vn, slots, P)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in pool]
    s = kvb.append_shape(tokens, kvh, D, P, pages, src)
    log(f"append of every {SRC[src]} row maximum: tokens={tokens} dim={D} page={P}")
    kvb.append_kv(s, kbuf.to(gpu), vbuf.to(gpu), torch.from_numpy(slots.view(np.int32)).to(gpu), *dev)
    torch.cuda.synchronize()
    for name, g, w in zip(("k", "v", "k_scales", "v_scales"), dev, want):
        got = g.cpu().numpy()
        assert np.array_equal(got.view(np.uint8) if got.dtype == np.int8 else got.view(np.uint32),
                              w.view(np.uint8) if w.dtype == np.int8 else w.view(np.uint32)), f"{name} differs"


def test_cache_written_by_append_decodes(gpu):
    """Prefill a cfg2-shaped (shorter) cache through three append calls; it
    equals the synthetic generator's cache bitwise and decodes to FP64."""
    import torch

    T, kvh, D, P, qh = 8192, 8, 128, 64, 32
    case = W.synth_case(1, qh, kvh, D, P, T, seed=123)
    pages = case.shape.pages
    # recover the fp32 source rows of the generator (same seed, same draws)
    rng = np.random.default_rng(123)
    _q = rng.standard_normal(qh * D, dtype=np.float32)
    kx = rng.standard_normal((pages, kvh, P, D), dtype=np.float32)
    vx = rng.standard_normal((pages, kvh, P, D), dtype=np.float32)
    # logical token t lives in physical page table[t // P], slot t % P; the
    # generator drew rows per physical (page, kv, slot)
    table = case.table.astype(np.int64)
    t = np.arange(T)
    phys = table[t // P]
    kn = kx[phys, :, t % P, :]                       # [T, kv, D]
    vn = vx[phys, :, t % P, :]
    slots = (phys * P + t % P).astype(np.uint32)
    dev_k = torch.zeros(case.k.shape, dtype=torch.int8, device=gpu)
    dev_v = torch.zeros(case.v.shape, dtype=torch.int8, device=gpu)
    dev_ks = torch.zeros(case.ks.shape, dtype=torch.float32, device=gpu)
    dev_vs = torch.zeros(case.vs.shape, dtype=torch.float32, device=gpu)
    kn_d = torch.from_numpy(np.ascontiguousarray(kn)).to(gpu)
    vn_d = torch.from_numpy(np.ascontiguousarray(vn)).to(gpu)
    sl_d = torch.from_numpy(slots.view(np.int32)).to(gpu)
    for lo, hi in ((0, 1000), (1000, 1001), (1001, T)):   # prefill chunks incl. a single-token step
        s = kvb.append_shape(hi - lo, kvh, D, P, pages)
        kvb.append_kv(s, kn_d[lo:hi], vn_d[lo:hi], sl_d[lo:hi], dev_k, dev_v, dev_ks, dev_vs)
    torch.cuda.synchronize()
    assert np.array_equal(dev_k.cpu().numpy(), case.k), "K pool differs from the generator's"
    assert np.array_equal(dev_v.cpu().numpy(), case.v), "V pool differs from the generator's"
    assert np.array_equal(dev_ks.cpu().numpy(), case.ks) and np.array_equal(dev_vs.cpu().numpy(), case.vs)
    dc = DeviceCase(case)
    dc.t.update(k=dev_k, v=dev_v, ks=dev_ks, vs=dev_vs)
    dc.inp = kvb.device_input(dc.t["q"], dc.t["qpos"], dc.t["kpos"], dc.t["table"], dev_k, dev_v, dev_ks, dev_vs)
    mln, _, _ = dc.run_decode(2048)
    check_against_oracle(case, mln, "decode of the appended cache")


def test_append_rejections(gpu):
    import torch

    s = kvb.append_shape(4, 8, 128, 64, 10)
    buf = torch.zeros(4 * 8 * 128, dtype=torch.float32, device=gpu)
    sl = torch.zeros(4, dtype=torch.int32, device=gpu)
    with pytest.raises(kvb.KvbInvalidArgument, match="non-null"):
        kvb.append_kv(s, buf, buf, sl, None, buf, buf, buf)
    with pytest.raises(kvb.KvbInvalidArgument, match="stride"):
        kvb.append_kv(kvb.append_shape(4, 8, 128, 64, 10, k_stride=100), buf, buf, sl, buf, buf, buf, buf)
    kvb.append_kv(kvb.append_shape(0, 8, 128, 64, 10), None, None, None, None, None, None, None)  # no-op
