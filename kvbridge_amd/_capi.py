"""ctypes binding of the C ABI in include/kvbridge_c.h (libkvbridge_amd.so).

This module only describes the extern "C" surface; it performs no arithmetic.
Loading fails loudly when the built library is missing: there is no CPU or
PyTorch fallback behind these entry points.
"""
from __future__ import annotations

import ctypes
import os

LIB_NAME = "libkvbridge_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

KVB_OK, KVB_EINVAL, KVB_ERUNTIME = 0, 1, 2
KVB_OUT_NONE, KVB_OUT_F32, KVB_OUT_F16 = 0, 1, 2
KVB_KERNEL_TILED_MFMA, KVB_KERNEL_GENERIC = 1, 2
KVB_SRC_F32, KVB_SRC_F16, KVB_SRC_BF16 = 1, 2, 3


class Shape(ctypes.Structure):
    """kvb_shape: mirrors kvbridge::Shape (reference include/kvbridge/attention_shape.h:9-13)."""

    _fields_ = [
        ("rows", ctypes.c_uint32),
        ("q_heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("dim", ctypes.c_uint32),
        ("page_tokens", ctypes.c_uint32),
        ("pages", ctypes.c_uint32),
        ("tokens", ctypes.c_uint32),
        ("begin", ctypes.c_uint32),
        ("end", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("int8", ctypes.c_uint32),
    ]

    def as_tuple(self):
        return tuple(getattr(self, f) for f, _ in self._fields_)

    def copy(self, **changes) -> "Shape":
        vals = {f: getattr(self, f) for f, _ in self._fields_}
        vals.update(changes)
        return Shape(**vals)


class DeviceInput(ctypes.Structure):
    """kvb_device_input: mirrors kvbridge::DeviceInput (reference attention_common.h:54-63)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_positions", ctypes.c_void_p),
        ("k_positions", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_scales", ctypes.c_void_p),
        ("v_scales", ctypes.c_void_p),
    ]


class BatchShape(ctypes.Structure):
    """kvb_batch_shape: mirrors kvbridge::BatchShape (include/kvbridge/attention_ext.h)."""

    _fields_ = [(n, ctypes.c_uint32) for n in
                ("batch", "rows", "q_heads", "kv_heads", "dim", "page_tokens", "pages",
                 "max_tokens", "total_tokens", "table_entries", "split_tokens")] + \
               [("scale", ctypes.c_float), ("int8", ctypes.c_uint32)]

    def as_tuple(self):
        return tuple(getattr(self, f) for f, _ in self._fields_)

    def copy(self, **changes) -> "BatchShape":
        vals = {f: getattr(self, f) for f, _ in self._fields_}
        vals.update(changes)
        return BatchShape(**vals)


class BatchInput(ctypes.Structure):
    """kvb_batch_input: mirrors kvbridge::BatchInput (include/kvbridge/attention_ext.h)."""

    _fields_ = [(n, ctypes.c_void_p) for n in
                ("q", "q_positions", "seq_starts", "page_offsets", "k_positions", "page_table",
                 "k", "v", "k_scales", "v_scales")]


class AppendShape(ctypes.Structure):
    """kvb_append_shape (include/kvbridge_c.h)."""

    _fields_ = [(n, ctypes.c_uint32) for n in
                ("tokens", "kv_heads", "dim", "page_tokens", "pages", "k_stride", "v_stride", "src_type")]


class AppendIO(ctypes.Structure):
    """kvb_append_io (include/kvbridge_c.h)."""

    _fields_ = [(n, ctypes.c_void_p) for n in ("k_new", "v_new", "slots", "k", "v", "k_scales", "v_scales")]


class KvbError(Exception):
    """Base class; the subclasses mirror std::invalid_argument / std::runtime_error."""


class KvbInvalidArgument(KvbError, ValueError):
    pass


class KvbRuntimeError(KvbError, RuntimeError):
    pass


# (name, restype, argtypes) for every function declared in include/kvbridge_c.h.
_SP = ctypes.POINTER(Shape)
_IP = ctypes.POINTER(DeviceInput)
_BSP = ctypes.POINTER(BatchShape)
_BIP = ctypes.POINTER(BatchInput)
_VP = ctypes.c_void_p
_U32 = ctypes.c_uint32
_INT = ctypes.c_int
SIGNATURES = [
    ("kvb_last_error", ctypes.c_char_p, []),
    ("kvb_split_tokens", _U32, []),
    ("kvb_shape_error", ctypes.c_char_p, [_SP]),
    ("kvb_shape_valid", _INT, [_SP]),
    ("kvb_split_count", _INT, [_SP, ctypes.POINTER(_U32)]),
    ("kvb_scratch_elements", _INT, [_SP, ctypes.POINTER(ctypes.c_size_t)]),
    ("kvb_output_scalar_elements", _INT, [_SP, ctypes.POINTER(ctypes.c_size_t)]),
    ("kvb_output_numerator_elements", _INT, [_SP, ctypes.POINTER(ctypes.c_size_t)]),
    ("kvb_mma_supported", _INT, [_SP]),
    ("kvb_preload_attention_kernels", _INT, []),
    ("kvb_preload_attention_reference_kernels", _INT, []),
    ("kvb_preload_attention_mma_kernels", _INT, []),
    ("kvb_launch_attention", _INT, [_SP, _IP, _VP, _VP, _VP, _VP, _VP]),
    ("kvb_launch_attention_mma", _INT, [_SP, _IP, _VP, _VP, _VP, _VP, _VP]),
    ("kvb_merge_attention", _INT, [_SP, _VP, _U32, _VP, _VP, _VP, _VP]),
    ("kvb_split_count_ex", _INT, [_SP, _U32, ctypes.POINTER(_U32)]),
    ("kvb_scratch_elements_ex", _INT, [_SP, _U32, ctypes.POINTER(ctypes.c_size_t)]),
    ("kvb_split_attention", _INT, [_SP, _IP, _U32, _VP, _VP]),
    ("kvb_merge_finalize", _INT, [_SP, _VP, _U32, _VP, _VP, _VP, _VP, _INT, _VP]),
    ("kvb_decode_attention", _INT, [_SP, _IP, _U32, _VP, _VP, _VP, _VP, _VP, _INT, _VP]),
    ("kvb_decode_attention_fused", _INT, [_SP, _IP, _U32, _VP, _VP, _VP, _VP, _VP, _VP, _INT, _VP]),
    ("kvb_decode_attention_fused_fenced", _INT, [_SP, _IP, _U32, _VP, _VP, _VP, _VP, _VP, _VP, _INT, _VP]),
    ("kvb_decode_attention_noalloc", _INT, [_SP, _IP, _U32, _VP, _VP, _VP, _VP, _INT, _VP]),
    ("kvb_selected_kernel", _INT, [_SP, _IP, _U32]),
    ("kvb_selected_kernel_name", ctypes.c_char_p, [_SP, _IP, _U32, _INT]),
    ("kvb_hbm_read_probe", _INT, [_VP, ctypes.c_size_t, _VP, _U32, _VP]),
    ("kvb_paged_read_probe", _INT, [_SP, _IP, _U32, _VP, _VP]),
    ("kvb_batch_shape_error", ctypes.c_char_p, [_BSP]),
    ("kvb_batch_split_count", _INT, [_BSP, ctypes.POINTER(_U32)]),
    ("kvb_batch_scratch_elements", _INT, [_BSP, ctypes.POINTER(ctypes.c_size_t)]),
    ("kvb_batch_output_scalar_elements", _INT, [_BSP, ctypes.POINTER(ctypes.c_size_t)]),
    ("kvb_decode_attention_batched", _INT, [_BSP, _BIP, _VP, _VP, _VP, _VP, _VP, _VP, _INT, _VP]),
    ("kvb_batch_kernel_name", ctypes.c_char_p, [_BSP, _BIP, _INT]),
    ("kvb_append_shape_error", ctypes.c_char_p, [ctypes.POINTER(AppendShape)]),
    ("kvb_append_kv", _INT, [ctypes.POINTER(AppendShape), ctypes.POINTER(AppendIO), _VP]),
]

_lib = None


def load() -> ctypes.CDLL:
    """Load libkvbridge_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, restype, argtypes in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def check(rc: int) -> None:
    """Raise the exception type matching a kvb_* status code."""
    if rc == KVB_OK:
        return
    msg = load().kvb_last_error().decode()
    if rc == KVB_EINVAL:
        raise KvbInvalidArgument(msg)
    raise KvbRuntimeError(msg)
