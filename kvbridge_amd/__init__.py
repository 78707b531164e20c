"""MI355X (gfx950) paged INT8-KV grouped-query split-K decode attention.

Python face of libkvbridge_amd.so.  Every call goes through the extern "C"
layer declared in include/kvbridge_c.h; PyTorch only provides device memory
and the HIP stream.  Names follow the reference C++ API (reference
include/kvbridge/attention_shape.h, attention_common.h): shape validation and
sizing, launch_attention, launch_attention_mma, merge_attention, preload_*,
plus the additive extensions (explicit split size, merge + normalize,
decode_attention).
"""
from __future__ import annotations

import ctypes

from ._capi import (  # noqa: F401
    KVB_SRC_BF16,
    KVB_SRC_F16,
    KVB_SRC_F32,
    AppendIO,
    AppendShape,
    BatchInput,
    BatchShape,
    KVB_KERNEL_GENERIC,
    KVB_KERNEL_TILED_MFMA,
    KVB_OUT_F16,
    KVB_OUT_F32,
    KVB_OUT_NONE,
    DeviceInput,
    KvbError,
    KvbInvalidArgument,
    KvbRuntimeError,
    Shape,
    check,
    load,
)

K_SPLIT_TOKENS = 256  # kvbridge::kSplitTokens (reference attention_shape.h:7)


def make_shape(rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end, scale, int8=True) -> Shape:
    return Shape(rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end, float(scale), 1 if int8 else 0)


# ---- host-only shape API (reference src/attention_shape.cpp) ----------------

def attention_shape_error(s: Shape):
    r = load().kvb_shape_error(ctypes.byref(s))
    return None if r is None else r.decode()


def attention_shape_valid(s: Shape) -> bool:
    return bool(load().kvb_shape_valid(ctypes.byref(s)))


def validate_shape(s: Shape) -> None:
    err = attention_shape_error(s)
    if err is not None:
        raise KvbInvalidArgument(err)


def split_count(s: Shape, split_tokens: int | None = None) -> int:
    out = ctypes.c_uint32()
    if split_tokens is None:
        check(load().kvb_split_count(ctypes.byref(s), ctypes.byref(out)))
    else:
        check(load().kvb_split_count_ex(ctypes.byref(s), split_tokens, ctypes.byref(out)))
    return out.value


def scratch_elements(s: Shape, split_tokens: int | None = None) -> int:
    out = ctypes.c_size_t()
    if split_tokens is None:
        check(load().kvb_scratch_elements(ctypes.byref(s), ctypes.byref(out)))
    else:
        check(load().kvb_scratch_elements_ex(ctypes.byref(s), split_tokens, ctypes.byref(out)))
    return out.value


def output_scalar_elements(s: Shape) -> int:
    out = ctypes.c_size_t()
    check(load().kvb_output_scalar_elements(ctypes.byref(s), ctypes.byref(out)))
    return out.value


def output_numerator_elements(s: Shape) -> int:
    out = ctypes.c_size_t()
    check(load().kvb_output_numerator_elements(ctypes.byref(s), ctypes.byref(out)))
    return out.value


def attention_mma_supported(s: Shape) -> bool:
    return bool(load().kvb_mma_supported(ctypes.byref(s)))


# ---- device entry points --------------------------------------------------

def preload_attention_kernels() -> int:
    return load().kvb_preload_attention_kernels()


def preload_attention_reference_kernels() -> int:
    return load().kvb_preload_attention_reference_kernels()


def preload_attention_mma_kernels() -> int:
    return load().kvb_preload_attention_mma_kernels()


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def device_input(q, q_positions, k_positions, page_table, k, v, k_scales=None, v_scales=None) -> DeviceInput:
    """Build a kvb_device_input from device tensors (or raw integer pointers)."""
    return DeviceInput(*(_ptr(x) for x in (q, q_positions, k_positions, page_table, k, v, k_scales, v_scales)))


def _stream(stream) -> int | None:
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def launch_attention(s: Shape, inp: DeviceInput, scratch, m, l, n, stream=None) -> None:
    check(load().kvb_launch_attention(ctypes.byref(s), ctypes.byref(inp), _ptr(scratch), _ptr(m), _ptr(l), _ptr(n), _stream(stream)))


def launch_attention_mma(s: Shape, inp: DeviceInput, scratch, m, l, n, stream=None) -> None:
    check(load().kvb_launch_attention_mma(ctypes.byref(s), ctypes.byref(inp), _ptr(scratch), _ptr(m), _ptr(l), _ptr(n), _stream(stream)))


def merge_attention(s: Shape, scratch, splits: int, m, l, n, stream=None) -> None:
    check(load().kvb_merge_attention(ctypes.byref(s), _ptr(scratch), splits, _ptr(m), _ptr(l), _ptr(n), _stream(stream)))


def split_attention(s: Shape, inp: DeviceInput, split_tokens: int, scratch, stream=None) -> None:
    check(load().kvb_split_attention(ctypes.byref(s), ctypes.byref(inp), split_tokens, _ptr(scratch), _stream(stream)))


def merge_finalize(s: Shape, scratch, splits: int, m, l, n, out=None, out_type: int = KVB_OUT_NONE, stream=None) -> None:
    check(load().kvb_merge_finalize(ctypes.byref(s), _ptr(scratch), splits, _ptr(m), _ptr(l), _ptr(n), _ptr(out), out_type, _stream(stream)))


def decode_attention(s: Shape, inp: DeviceInput, split_tokens: int, scratch, m, l, n, out=None,
                     out_type: int = KVB_OUT_NONE, stream=None) -> None:
    check(load().kvb_decode_attention(ctypes.byref(s), ctypes.byref(inp), split_tokens, _ptr(scratch), _ptr(m), _ptr(l),
                                      _ptr(n), _ptr(out), out_type, _stream(stream)))


def decode_attention_fused(s: Shape, inp: DeviceInput, split_tokens: int, scratch, counters, m, l, n, out=None,
                           out_type: int = KVB_OUT_NONE, stream=None) -> None:
    """Single-launch decode (kvb_decode_attention_fused): `counters` is a
    device uint32 buffer of kv_heads zeros, left zero by every call."""
    check(load().kvb_decode_attention_fused(ctypes.byref(s), ctypes.byref(inp), split_tokens, _ptr(scratch),
                                            _ptr(counters), _ptr(m), _ptr(l), _ptr(n), _ptr(out), out_type,
                                            _stream(stream)))


def decode_attention_fused_fenced(s: Shape, inp: DeviceInput, split_tokens: int, scratch, counters, m, l, n,
                                  out=None, out_type: int = KVB_OUT_NONE, stream=None) -> None:
    """Diagnostic (kvb_decode_attention_fused_fenced): the single launch with
    formal release / acquire fences around the merge ticket; bitwise the
    same results as decode_attention_fused."""
    check(load().kvb_decode_attention_fused_fenced(ctypes.byref(s), ctypes.byref(inp), split_tokens, _ptr(scratch),
                                                   _ptr(counters), _ptr(m), _ptr(l), _ptr(n), _ptr(out), out_type,
                                                   _stream(stream)))


def decode_attention_noalloc(s: Shape, inp: DeviceInput, split_tokens: int, m, l, n, out=None,
                             out_type: int = KVB_OUT_NONE, stream=None) -> None:
    """Single-launch decode with the library's fixed 8 MiB per-device scratch
    (kvb_decode_attention_noalloc): no caller scratch or counters, no allocation."""
    check(load().kvb_decode_attention_noalloc(ctypes.byref(s), ctypes.byref(inp), split_tokens, _ptr(m), _ptr(l),
                                              _ptr(n), _ptr(out), out_type, _stream(stream)))


def selected_kernel(s: Shape, inp: DeviceInput, split_tokens: int) -> int:
    return load().kvb_selected_kernel(ctypes.byref(s), ctypes.byref(inp), split_tokens)


def selected_kernel_name(s: Shape, inp: DeviceInput, split_tokens: int, fused: bool = False) -> str:
    return load().kvb_selected_kernel_name(ctypes.byref(s), ctypes.byref(inp), split_tokens, int(fused)).decode()


def hbm_read_probe(src, nbytes: int, sink, blocks: int, stream=None) -> None:
    """Diagnostic streaming read of nbytes of device memory (see kvb_hbm_read_probe)."""
    check(load().kvb_hbm_read_probe(_ptr(src), nbytes, _ptr(sink), blocks, _stream(stream)))


def paged_read_probe(s: Shape, inp: DeviceInput, split_tokens: int, sink, stream=None) -> None:
    """Diagnostic read of a decode call's KV bytes through its page table (see kvb_paged_read_probe)."""
    check(load().kvb_paged_read_probe(ctypes.byref(s), ctypes.byref(inp), split_tokens, _ptr(sink), _stream(stream)))


# ---- batched ragged decode (kvb_decode_attention_batched) ---------------------

def make_batch_shape(batch, rows, q_heads, kv_heads, dim, page_tokens, pages, max_tokens, total_tokens,
                     table_entries, split_tokens, scale, int8=True) -> BatchShape:
    return BatchShape(batch, rows, q_heads, kv_heads, dim, page_tokens, pages, max_tokens, total_tokens,
                      table_entries, split_tokens, float(scale), 1 if int8 else 0)


def batch_shape_error(s: BatchShape):
    r = load().kvb_batch_shape_error(ctypes.byref(s))
    return None if r is None else r.decode()


def batch_split_count(s: BatchShape) -> int:
    out = ctypes.c_uint32()
    check(load().kvb_batch_split_count(ctypes.byref(s), ctypes.byref(out)))
    return out.value


def batch_scratch_elements(s: BatchShape) -> int:
    out = ctypes.c_size_t()
    check(load().kvb_batch_scratch_elements(ctypes.byref(s), ctypes.byref(out)))
    return out.value


def batch_output_scalar_elements(s: BatchShape) -> int:
    out = ctypes.c_size_t()
    check(load().kvb_batch_output_scalar_elements(ctypes.byref(s), ctypes.byref(out)))
    return out.value


def batch_input(q, q_positions, seq_starts, page_offsets, k_positions, page_table, k, v, k_scales=None,
                v_scales=None) -> BatchInput:
    """Build a kvb_batch_input from device tensors (or raw integer pointers)."""
    return BatchInput(*(_ptr(x) for x in (q, q_positions, seq_starts, page_offsets, k_positions, page_table,
                                          k, v, k_scales, v_scales)))


def decode_attention_batched(s: BatchShape, inp: BatchInput, scratch, m, l, n, out=None,
                             out_type: int = KVB_OUT_NONE, counters=None, stream=None) -> None:
    """Batched decode (kvb_decode_attention_batched): one launch when `counters`
    (batch * kv_heads uint32 zeros, left zero) is given and the int8 kernel
    serves the shape, else split + merge launches."""
    check(load().kvb_decode_attention_batched(ctypes.byref(s), ctypes.byref(inp), _ptr(scratch), _ptr(counters),
                                              _ptr(m), _ptr(l), _ptr(n), _ptr(out), out_type, _stream(stream)))


def batch_kernel_name(s: BatchShape, inp: BatchInput, fused: bool = False) -> str:
    return load().kvb_batch_kernel_name(ctypes.byref(s), ctypes.byref(inp), int(fused)).decode()


# ---- paged INT8 KV append (kvb_append_kv) ---------------------------------------

def append_shape(tokens, kv_heads, dim, page_tokens, pages, src_type=KVB_SRC_F32, k_stride=None,
                 v_stride=None) -> AppendShape:
    row = kv_heads * dim
    return AppendShape(tokens, kv_heads, dim, page_tokens, pages, row if k_stride is None else k_stride,
                       row if v_stride is None else v_stride, src_type)


def append_shape_error(s: AppendShape):
    r = load().kvb_append_shape_error(ctypes.byref(s))
    return None if r is None else r.decode()


def append_kv(s: AppendShape, k_new, v_new, slots, k, v, k_scales, v_scales, stream=None) -> None:
    """Quantize new tokens' K/V rows into their physical slots of the pool
    (kvb_append_kv): per-(token, kv head) absmax scales, K token-major, V
    dim-major."""
    io = AppendIO(*(_ptr(x) for x in (k_new, v_new, slots, k, v, k_scales, v_scales)))
    check(load().kvb_append_kv(ctypes.byref(s), ctypes.byref(io), _stream(stream)))
