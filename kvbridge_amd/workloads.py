"""Seeded synthetic paged INT8-KV decode workloads.

Builds the cache in the library's HBM layout (include/kvbridge/attention_common.h):
  K int8 [pages, kv_heads, page_tokens, dim]   token-major
  V int8 [pages, kv_heads, dim, page_tokens]   dim-major
  k/v scales fp32 [pages, kv_heads, page_tokens]
Q is drawn N(0,1) and rounded to fp16 (stored as fp32, so it is fp16-exact).
K/V values are drawn N(0,1) per physical (page, kv_head, slot, dim) and
quantised per (token, kv_head) to symmetric int8: scale = absmax / 127
(scale 1 and codes 0 for an all-zero row), code = clamp(rint(x / scale),
-127, 127).  The page table is a seeded permutation of the page pool.

numpy generators serve the CPU-checked parity cases; the torch generators
build large caches directly in device memory for the benchmark.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from ._capi import BatchShape, Shape


@dataclass
class Case:
    shape: Shape
    q: np.ndarray          # float32 [rows*q_heads*dim]
    qpos: np.ndarray       # int64 [rows]
    kpos: np.ndarray       # int64 [tokens]
    table: np.ndarray      # uint32 [pages]
    k: np.ndarray          # int8 (or float32) [pages, kv, P, D]
    v: np.ndarray          # int8 (or float32) [pages, kv, D, P]
    ks: np.ndarray         # float32 [pages, kv, P]
    vs: np.ndarray         # float32 [pages, kv, P]
    meta: dict = field(default_factory=dict)

    def kv_bytes(self) -> int:
        """Algorithmic KV bytes of one call: int8 K + V and fp32 k/v scales of [begin, end)."""
        s = self.shape
        return (s.end - s.begin) * s.kv_heads * (2 * s.dim + 8)

    def to_device(self, device="cuda"):
        import torch

        return {
            "q": torch.from_numpy(self.q).to(device),
            "qpos": torch.from_numpy(self.qpos).to(device),
            "kpos": torch.from_numpy(self.kpos).to(device),
            "table": torch.from_numpy(self.table.view(np.int32)).to(device),
            "k": torch.from_numpy(np.ascontiguousarray(self.k)).to(device),
            "v": torch.from_numpy(np.ascontiguousarray(self.v)).to(device),
            "ks": torch.from_numpy(self.ks).to(device),
            "vs": torch.from_numpy(self.vs).to(device),
        }


def quantize_rows(x: np.ndarray):
    """Per-row (last axis) symmetric int8: returns (codes int8, scales float32)."""
    absmax = np.max(np.abs(x), axis=-1)
    scale = (absmax / np.float32(127)).astype(np.float32)
    scale = np.where(absmax == 0, np.float32(1), scale).astype(np.float32)
    codes = np.clip(np.rint(x / scale[..., None]), -127, 127).astype(np.int8)
    return codes, scale


def synth_case(rows, q_heads, kv_heads, dim, page_tokens, tokens, *, seed, pages=None, permute=True,
               scale=None, begin=0, end=None, qpos=None, kpos=None, outlier_frac=0.0, outlier_mult=8.0,
               int8=True) -> Case:
    rng = np.random.default_rng(seed)
    pages = pages if pages is not None else -(-tokens // page_tokens)
    end = tokens if end is None else end
    scale = 1.0 / math.sqrt(dim) if scale is None else scale
    q = rng.standard_normal(rows * q_heads * dim, dtype=np.float32).astype(np.float16).astype(np.float32)
    kx = rng.standard_normal((pages, kv_heads, page_tokens, dim), dtype=np.float32)
    vx = rng.standard_normal((pages, kv_heads, page_tokens, dim), dtype=np.float32)
    if outlier_frac > 0:
        hit = rng.random((pages, 1, page_tokens, 1)) < outlier_frac
        mult = np.where(hit, np.float32(outlier_mult), np.float32(1))
        kx *= mult
        vx *= mult
    if int8:
        k, ks = quantize_rows(kx)
        vq, vs = quantize_rows(vx)
    else:
        k, vq = kx, vx
        ks = np.ones((pages, kv_heads, page_tokens), np.float32)
        vs = np.ones((pages, kv_heads, page_tokens), np.float32)
    v = np.ascontiguousarray(vq.transpose(0, 1, 3, 2))
    table = (rng.permutation(pages) if permute else np.arange(pages)).astype(np.uint32)
    kpos = np.arange(tokens, dtype=np.int64) if kpos is None else np.asarray(kpos, np.int64)
    qpos = (np.arange(rows, dtype=np.int64) + tokens - rows) if qpos is None else np.asarray(qpos, np.int64)
    shape = Shape(rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end, float(scale), 1 if int8 else 0)
    return Case(shape, q, qpos, kpos, table, np.ascontiguousarray(k), v, ks, vs,
                meta={"seed": seed, "permute": permute, "outlier_frac": outlier_frac})


# ---- BASELINE.json configurations -------------------------------------------

def cfg1(seed=0x4B56421) -> tuple[Case, int]:
    """1 seq, 8q/2kv, d64, 512 tokens, page 16, pages in order; split-K 4 chunks."""
    return synth_case(1, 8, 2, 64, 16, 512, seed=seed, permute=False), 128


def cfg2(seed=0x4B56422) -> tuple[Case, int]:
    """1 seq, 32q/8kv, d128, 65536 tokens, page 64, random permutation of 1024 pages; 32 splits."""
    return synth_case(1, 32, 8, 128, 64, 65536, seed=seed, permute=True), 2048


def torch_cache(rows, q_heads, kv_heads, dim, page_tokens, tokens, *, seed, device="cuda", outlier_frac=0.0,
                outlier_mult=8.0):
    """Same distribution as synth_case, generated in device memory with torch."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pages = -(-tokens // page_tokens)
    q = torch.randn(rows * q_heads * dim, generator=g, device=device).half().float()
    out = {"q": q}
    for name in ("k", "v"):
        x = torch.randn((pages, kv_heads, page_tokens, dim), generator=g, device=device)
        if outlier_frac > 0:
            hit = torch.rand((pages, 1, page_tokens, 1), generator=g, device=device) < outlier_frac
            x = torch.where(hit, x * outlier_mult, x)
        absmax = x.abs().amax(dim=-1)
        sc = absmax / 127.0
        sc = torch.where(absmax == 0, torch.ones_like(sc), sc)
        codes = torch.clamp(torch.round(x / sc[..., None]), -127, 127).to(torch.int8)
        if name == "v":
            codes = codes.transpose(2, 3).contiguous()
        out[name] = codes.contiguous()
        out[name + "s"] = sc.contiguous()
        del x
    out["table"] = torch.randperm(pages, generator=g, device=device).to(torch.int32)
    out["kpos"] = torch.arange(tokens, dtype=torch.int64, device=device)
    out["qpos"] = torch.arange(rows, dtype=torch.int64, device=device) + tokens - rows
    shape = Shape(rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, 0, tokens, 1.0 / math.sqrt(dim), 1)
    return shape, out


# ---- batched ragged workloads (kvb_decode_attention_batched) -----------------

@dataclass
class BatchCase:
    """A batch of sequences over one shared page pool (host arrays)."""
    shape: BatchShape
    q: np.ndarray             # float32 [batch*rows*q_heads*dim]
    qpos: np.ndarray          # int64 [batch*rows]
    seq_starts: np.ndarray    # uint32 [batch+1]
    page_offsets: np.ndarray  # uint32 [batch]
    kpos: np.ndarray          # int64 [total_tokens]
    table: np.ndarray         # uint32 [table_entries]
    k: np.ndarray
    v: np.ndarray
    ks: np.ndarray
    vs: np.ndarray
    lengths: list = field(default_factory=list)

    def kv_bytes(self) -> int:
        s = self.shape
        return int(sum(self.lengths)) * s.kv_heads * (2 * s.dim + 8)

    def sequence(self, b: int) -> Case:
        """Sequence b as a single-sequence Case over the same pool (tokens [0, T_b))."""
        s = self.shape
        t0, t1 = int(self.seq_starts[b]), int(self.seq_starts[b + 1])
        T = t1 - t0
        np_ = -(-T // s.page_tokens)
        off = int(self.page_offsets[b])
        rh = s.rows * s.q_heads * s.dim
        shape = Shape(s.rows, s.q_heads, s.kv_heads, s.dim, s.page_tokens, s.pages, T, 0, T, s.scale, s.int8)
        return Case(shape, self.q[b * rh:(b + 1) * rh], self.qpos[b * s.rows:(b + 1) * s.rows],
                    self.kpos[t0:t1], np.ascontiguousarray(self.table[off:off + np_]), self.k, self.v, self.ks,
                    self.vs)

    def to_device(self, device="cuda"):
        import torch

        return {
            "q": torch.from_numpy(self.q).to(device),
            "qpos": torch.from_numpy(self.qpos).to(device),
            "starts": torch.from_numpy(self.seq_starts.view(np.int32)).to(device),
            "offsets": torch.from_numpy(self.page_offsets.view(np.int32)).to(device),
            "kpos": torch.from_numpy(self.kpos).to(device),
            "table": torch.from_numpy(self.table.view(np.int32)).to(device),
            "k": torch.from_numpy(np.ascontiguousarray(self.k)).to(device),
            "v": torch.from_numpy(np.ascontiguousarray(self.v)).to(device),
            "ks": torch.from_numpy(self.ks).to(device),
            "vs": torch.from_numpy(self.vs).to(device),
        }


def _batch_layout(lengths, page_tokens, rows, rng_perm):
    """Pool size, per-sequence page lists (slices of a shuffled pool), offsets, starts, positions."""
    lengths = [int(t) for t in lengths]
    npages = [-(-t // page_tokens) for t in lengths]
    pool = max(1, sum(npages))
    table = rng_perm(pool).astype(np.uint32)
    offsets = np.concatenate([[0], np.cumsum(npages)[:-1]]).astype(np.uint32)
    starts = np.concatenate([[0], np.cumsum(lengths)]).astype(np.uint32)
    kpos = np.concatenate([np.arange(t, dtype=np.int64) for t in lengths]) if sum(lengths) else \
        np.zeros(1, np.int64)
    qpos = np.concatenate([np.arange(rows, dtype=np.int64) + t - rows for t in lengths])
    return lengths, pool, table, offsets, starts, kpos, qpos


def synth_batch(rows, q_heads, kv_heads, dim, page_tokens, lengths, *, seed, split_tokens, outlier_frac=0.0,
                outlier_mult=8.0, int8=True, scale=None) -> BatchCase:
    """Ragged batch over a shuffled shared pool sized to the total token count (numpy, small cases)."""
    rng = np.random.default_rng(seed)
    lengths, pool, table, offsets, starts, kpos, qpos = _batch_layout(lengths, page_tokens, rows, rng.permutation)
    batch = len(lengths)
    scale = 1.0 / math.sqrt(dim) if scale is None else scale
    q = rng.standard_normal(batch * rows * q_heads * dim, dtype=np.float32).astype(np.float16).astype(np.float32)
    kx = rng.standard_normal((pool, kv_heads, page_tokens, dim), dtype=np.float32)
    vx = rng.standard_normal((pool, kv_heads, page_tokens, dim), dtype=np.float32)
    if outlier_frac > 0:
        hit = rng.random((pool, 1, page_tokens, 1)) < outlier_frac
        mult = np.where(hit, np.float32(outlier_mult), np.float32(1))
        kx *= mult
        vx *= mult
    if int8:
        k, ks = quantize_rows(kx)
        vq, vs = quantize_rows(vx)
    else:
        k, vq = kx, vx
        ks = np.ones((pool, kv_heads, page_tokens), np.float32)
        vs = np.ones((pool, kv_heads, page_tokens), np.float32)
    v = np.ascontiguousarray(vq.transpose(0, 1, 3, 2))
    shape = BatchShape(batch, rows, q_heads, kv_heads, dim, page_tokens, pool, max(1, max(lengths)), len(kpos),
                       len(table), split_tokens, float(scale), 1 if int8 else 0)
    return BatchCase(shape, q, qpos, starts, offsets, kpos, table, np.ascontiguousarray(k), v, ks, vs, lengths)


def torch_batch(rows, q_heads, kv_heads, dim, page_tokens, lengths, *, seed, split_tokens, device="cuda",
                outlier_frac=0.0, outlier_mult=8.0):
    """Same distribution as synth_batch, generated in device memory with torch (large configs)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    perm = np.random.default_rng(seed).permutation
    lengths, pool, table, offsets, starts, kpos, qpos = _batch_layout(lengths, page_tokens, rows, perm)
    batch = len(lengths)
    out = {"q": torch.randn(batch * rows * q_heads * dim, generator=g, device=device).half().float()}
    for name in ("k", "v"):
        codes = torch.empty((pool, kv_heads, page_tokens, dim), dtype=torch.int8, device=device)
        sc = torch.empty((pool, kv_heads, page_tokens), dtype=torch.float32, device=device)
        for p0 in range(0, pool, 1024):  # bounded temporaries
            p1 = min(pool, p0 + 1024)
            x = torch.randn((p1 - p0, kv_heads, page_tokens, dim), generator=g, device=device)
            if outlier_frac > 0:
                hit = torch.rand((p1 - p0, 1, page_tokens, 1), generator=g, device=device) < outlier_frac
                x = torch.where(hit, x * outlier_mult, x)
            absmax = x.abs().amax(dim=-1)
            s_ = torch.where(absmax == 0, torch.ones_like(absmax), absmax / 127.0)
            codes[p0:p1] = torch.clamp(torch.round(x / s_[..., None]), -127, 127).to(torch.int8)
            sc[p0:p1] = s_
            del x
        if name == "v":
            codes = codes.transpose(2, 3).contiguous()
        out[name] = codes
        out[name + "s"] = sc
    out["table"] = torch.from_numpy(table.view(np.int32)).to(device)
    out["offsets"] = torch.from_numpy(offsets.view(np.int32)).to(device)
    out["starts"] = torch.from_numpy(starts.view(np.int32)).to(device)
    out["kpos"] = torch.from_numpy(kpos).to(device)
    out["qpos"] = torch.from_numpy(qpos).to(device)
    shape = BatchShape(batch, rows, q_heads, kv_heads, dim, page_tokens, pool, max(1, max(lengths)), len(kpos),
                       len(table), split_tokens, 1.0 / math.sqrt(dim), 1)
    return shape, out, lengths


def batch_to_host(shape: BatchShape, t: dict, lengths) -> BatchCase:
    """Copy a torch_batch cache to host arrays (for the CPU oracle)."""
    return BatchCase(shape, t["q"].cpu().numpy(), t["qpos"].cpu().numpy(),
                     t["starts"].cpu().numpy().view(np.uint32), t["offsets"].cpu().numpy().view(np.uint32),
                     t["kpos"].cpu().numpy(), t["table"].cpu().numpy().view(np.uint32), t["k"].cpu().numpy(),
                     t["v"].cpu().numpy(), t["ks"].cpu().numpy(), t["vs"].cpu().numpy(), list(lengths))


def cfg3_lengths(seed=0x4B56423):
    """16 context lengths uniform in [1024, 32768]."""
    return [int(x) for x in np.random.default_rng(seed).integers(1024, 32768, size=16, endpoint=True)]


# configs[2] leaves the chunk count per sequence free ("chosen from its
# length"): ceil(length / 5120) chunks puts the batch's 57 chunks x 8 kv heads
# (456 work-groups) in one round of two work-groups per CU.  Measured on
# MI355X (split + merge, µs): 1024: 134, 1536: 101.5, 2048: 116.7, 3072: 99.5,
# 4096: 129, 4608: 101, 5120: 90.9, 6144: 95.5 -- a second, partly filled
# round of work-groups costs up to a third more.
CFG3 = dict(rows=1, q_heads=32, kv_heads=8, dim=128, page_tokens=64, split_tokens=5120)
CFG4 = dict(rows=1, q_heads=64, kv_heads=8, dim=128, page_tokens=64, split_tokens=2048,
            lengths=[131072] * 4, outlier_frac=0.01)
