"""Host-side shape/sizing API through the C ABI (no GPU needed).

Known-answer checks restate the reference's host test tests/shape_test.cpp
(:30-86): the same base shape, the same expected counts and the same reject
set, here exercised through kvb_* of libkvbridge_amd.so.  Validation order
and messages follow src/attention_shape.cpp:20-51.
"""
import math

import pytest

import kvbridge_amd as kvb

U32_MAX = 0xFFFFFFFF
BASE = dict(rows=8, q_heads=24, kv_heads=4, dim=256, page_tokens=32, pages=2048, tokens=65536, begin=0, end=65536,
            scale=0.0625, int8=1)


def shape(**kw):
    d = dict(BASE)
    d.update(kw)
    return kvb.Shape(**d)


def test_base_shape_counts():
    s = shape()
    assert kvb.attention_shape_valid(s)
    assert kvb.attention_shape_error(s) is None
    assert kvb.attention_mma_supported(s)
    assert kvb.split_count(s) == 256
    assert kvb.output_scalar_elements(s) == 192
    assert kvb.output_numerator_elements(s) == 49152
    assert kvb.scratch_elements(s) == 192 * 256 * 258
    assert kvb.K_SPLIT_TOKENS == kvb.load().kvb_split_tokens() == 256


REJECTS = [
    ("zero rows", dict(rows=0)),
    ("zero q heads", dict(q_heads=0)),
    ("zero kv heads", dict(kv_heads=0)),
    ("non-divisible heads", dict(q_heads=25)),
    ("more kv than q heads", dict(kv_heads=48)),
    ("zero dim", dict(dim=0)),
    ("dim beyond 256", dict(dim=257)),
    ("zero pages", dict(pages=0)),
    ("zero page tokens", dict(page_tokens=0)),
    ("zero backing tokens", dict(tokens=0, end=0)),
    ("reversed interval", dict(begin=33, end=32)),
    ("end past token storage", dict(end=65537)),
    ("token storage past page capacity", dict(pages=2047)),
    ("infinite scale", dict(scale=math.inf)),
    ("NaN scale", dict(scale=math.nan)),
    ("grid x product overflow", dict(rows=U32_MAX)),
    ("physical index overflow", dict(pages=U32_MAX)),
    ("head/storage products bounded", dict(kv_heads=0xFFFFFFFE, q_heads=0xFFFFFFFE)),
]


@pytest.mark.parametrize("label,change", REJECTS, ids=[r[0] for r in REJECTS])
def test_rejects(label, change):
    s = shape(**change)
    assert not kvb.attention_shape_valid(s), label
    assert kvb.attention_shape_error(s) is not None, label
    assert not kvb.attention_mma_supported(s), label
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.scratch_elements(s)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.split_count(s)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.validate_shape(s)


def test_intervals_and_mma_predicate():
    s = shape(begin=32, end=32)
    assert kvb.attention_shape_valid(s) and kvb.attention_mma_supported(s)
    assert kvb.split_count(s) == 1
    assert kvb.scratch_elements(s) == 192 * 258
    s = shape(begin=32, end=33)
    assert kvb.attention_mma_supported(s) and kvb.split_count(s) == 1
    s = shape(begin=32, end=289)
    assert kvb.split_count(s) == 2
    s = shape(begin=31, end=289)
    assert kvb.attention_shape_valid(s) and not kvb.attention_mma_supported(s)
    for change in (dict(int8=0), dict(rows=1), dict(dim=1), dict(q_heads=36)):
        s = shape(**change)
        assert kvb.attention_shape_valid(s) and not kvb.attention_mma_supported(s), change
    s = shape(tokens=65535, end=65535)
    assert kvb.attention_mma_supported(s)


def test_grid_y_limits():
    s = kvb.Shape(1, 1, 1, 1, 256, 65536, 16777216, 0, 16776960, 1.0, 1)
    assert kvb.split_count(s) == 65535
    s2 = s.copy(end=16776961)
    assert not kvb.attention_shape_valid(s2)
    assert "split" in kvb.attention_shape_error(s2)
    s = kvb.Shape(1, 1, 1, 1, 1, U32_MAX, U32_MAX, 0xFFFFFFFE, U32_MAX, 1.0, 1)
    assert kvb.split_count(s) == 1
    assert kvb.split_count(s.copy(begin=U32_MAX)) == 1


def test_first_failure_wins_and_messages():
    # Ordered checks: positivity before divisibility before dim before capacity.
    assert kvb.attention_shape_error(shape(rows=0, dim=0)) == "rows and head counts must be positive"
    assert "divisible" in kvb.attention_shape_error(shape(q_heads=25, dim=0))
    assert "dim" in kvb.attention_shape_error(shape(dim=257, pages=0))
    assert "scale" in kvb.attention_shape_error(shape(scale=math.nan))


def test_explicit_split_extension():
    s = kvb.Shape(1, 32, 8, 128, 64, 1024, 65536, 0, 65536, 1 / math.sqrt(128), 1)
    assert kvb.split_count(s, 2048) == 32
    assert kvb.scratch_elements(s, 2048) == 32 * 32 * 130
    assert kvb.split_count(s, 256) == kvb.split_count(s) == 256
    assert kvb.split_count(s, 100000) == 1
    assert kvb.split_count(s.copy(begin=5, end=5), 2048) == 1
    with pytest.raises(kvb.KvbInvalidArgument, match="split_tokens must be positive"):
        kvb.split_count(s, 0)
    # 65536 tokens in 1-token splits is over the 65535-split limit.
    with pytest.raises(kvb.KvbInvalidArgument, match="65535"):
        kvb.split_count(s, 1)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.split_count(s.copy(rows=0), 2048)


def test_launch_rejects_before_device_work():
    """Invalid metadata and null pointers are rejected on the host (no GPU
    call is made, so this runs without a device)."""
    s = kvb.Shape(1, 8, 2, 64, 16, 32, 512, 0, 512, 0.125, 1)
    inp = kvb.DeviceInput()
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.launch_attention(s.copy(rows=0), inp, 0, 0, 0, 0, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.launch_attention(s, inp, 0, 0, 0, 0, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.merge_attention(s, 0, 4, 0, 0, 0, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.decode_attention(s, inp, 0, 0, 0, 0, 0, stream=0)
    # Order of the reference checks (src/attention_launch_checks.h:8-23,
    # src/attention_mma.cu:36-40): outputs, inputs, alignment, then geometry.
    # The fake addresses below are never dereferenced: every call throws first.
    with pytest.raises(kvb.KvbInvalidArgument, match="scratch, m, l and n"):
        kvb.launch_attention(s, inp, 0x1000, 0, 0x1000, 0x1000, stream=0)
    fake = kvb.device_input(*([0x10000] * 8))
    with pytest.raises(kvb.KvbInvalidArgument, match="launch_attention_mma requires"):
        kvb.launch_attention_mma(s, fake, 0x1000, 0x1000, 0x1000, 0x1000, stream=0)
    misaligned = kvb.device_input(*([0x10000] * 4), 0x10002, 0x10000, 0x10000, 0x10000)
    with pytest.raises(kvb.KvbInvalidArgument, match="4-byte aligned"):
        kvb.launch_attention(s, misaligned, 0x1000, 0x1000, 0x1000, 0x1000, stream=0)
