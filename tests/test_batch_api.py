"""Host-side contract of the batched decode extension (no GPU): validation
order and messages, sizing, and argument rejection before any launch."""
import math

import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W


def cfg4_shape(**chg):
    s = kvb.make_batch_shape(4, 1, 64, 8, 128, 64, 8192, 131072, 4 * 131072, 8192, 2048, 1 / math.sqrt(128))
    return s.copy(**chg)


def test_valid_shapes_and_sizes():
    s = cfg4_shape()
    assert kvb.batch_shape_error(s) is None
    assert kvb.batch_split_count(s) == 64
    assert kvb.batch_scratch_elements(s) == 4 * 64 * 64 * 130
    assert kvb.batch_output_scalar_elements(s) == 4 * 64
    lens = W.cfg3_lengths()
    assert len(lens) == 16 and all(1024 <= t <= 32768 for t in lens)
    s3 = kvb.make_batch_shape(16, 1, 32, 8, 128, 64, sum(-(-t // 64) for t in lens), max(lens), sum(lens),
                              sum(-(-t // 64) for t in lens), 2048, 1 / math.sqrt(128))
    assert kvb.batch_shape_error(s3) is None
    assert kvb.batch_split_count(s3) == -(-max(lens) // 2048)


@pytest.mark.parametrize("change,msg", [
    (dict(batch=0), "batch must be in [1,65535]"),
    (dict(batch=65536), "batch must be in [1,65535]"),
    (dict(rows=0), "rows and head counts must be positive"),
    (dict(q_heads=60), "q_heads must be divisible by kv_heads"),
    (dict(dim=257), "dim must be in [1,256]"),
    (dict(max_tokens=0), "page_tokens, pages and tokens must be positive"),
    (dict(max_tokens=8192 * 64 + 1), "tokens exceed allocated page capacity"),
    (dict(scale=float("inf")), "score scale must be finite"),
    (dict(split_tokens=0), "split_tokens must be positive"),
    (dict(split_tokens=1), "split count exceeds 65535"),
    (dict(total_tokens=0), "total_tokens and table_entries must be positive"),
    (dict(table_entries=0), "total_tokens and table_entries must be positive"),
    (dict(batch=65535, rows=8, q_heads=8192, kv_heads=8), "batch row/head product exceeds the grid limit"),
])
def test_rejections_in_order(change, msg):
    s = cfg4_shape(**change)
    assert kvb.batch_shape_error(s) == msg
    with pytest.raises(kvb.KvbInvalidArgument, match=msg.replace("[", r"\[").replace("]", r"\]")):
        kvb.batch_split_count(s)


def test_call_rejected_before_launch():
    s = cfg4_shape()
    fake = 0x1000
    inp = kvb.batch_input(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake)
    with pytest.raises(kvb.KvbInvalidArgument, match="scratch, m, l and n"):
        kvb.decode_attention_batched(s, inp, None, fake, fake, fake, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument, match="attention input device buffers"):
        kvb.decode_attention_batched(s, kvb.batch_input(fake, fake, None, fake, fake, fake, fake, fake, fake, fake),
                                     fake, fake, fake, fake, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument, match="unknown output type"):
        kvb.decode_attention_batched(s, inp, fake, fake, fake, fake, fake, 7, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument, match="output buffer"):
        kvb.decode_attention_batched(s, inp, fake, fake, fake, fake, None, kvb.KVB_OUT_F16, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument, match="4-byte aligned"):
        kvb.decode_attention_batched(s, kvb.batch_input(fake, fake, fake, fake, fake, fake, fake + 1, fake, fake,
                                                        fake), fake, fake, fake, fake, stream=0)
    with pytest.raises(kvb.KvbInvalidArgument, match="batch must be"):
        kvb.decode_attention_batched(s.copy(batch=0), inp, fake, fake, fake, fake, stream=0)


def test_kernel_choice_names():
    s = cfg4_shape()
    fake = 0x1000
    inp = kvb.batch_input(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake)
    # 4 x 64 splits x 8 kv heads = 2048 work-groups of 32-tile splits -> one wave per
    # work-group, no single launch (more than two work-groups per CU): split + merge kernels
    assert kvb.batch_kernel_name(s, inp, fused=True) == "split_i8_kernel<128,1,2,true,8,false,true,false>"
    assert kvb.batch_kernel_name(s, inp) == "split_i8_kernel<128,1,2,true,8,false,true,false>"
    # one sequence: 512 work-groups -> four-wave groups
    assert kvb.batch_kernel_name(s.copy(batch=1), inp) == "split_i8_kernel<128,4,2,true,8,false,true,false>"
    # 4 head-rows, 2048 work-groups of 32-tile splits -> one wave, two launches;
    # 512 work-groups -> eight-wave single launch; 256 -> eight waves
    g4 = s.copy(q_heads=32)
    assert kvb.batch_kernel_name(g4, inp) == "split_i8_kernel<128,1,2,true,4,false,true,false>"
    assert kvb.batch_kernel_name(g4, inp, fused=True) == "split_i8_kernel<128,1,2,true,4,false,true,false>"
    assert kvb.batch_kernel_name(g4.copy(batch=16, max_tokens=32768), inp, fused=True) == \
        "split_i8_kernel<128,1,2,true,4,false,true,false>"
    # 2048 work-groups of 80-tile splits -> four waves
    assert kvb.batch_kernel_name(g4.copy(batch=16, max_tokens=81920, split_tokens=5120), inp) == \
        "split_i8_kernel<128,4,2,true,4,false,true,false>"
    assert kvb.batch_kernel_name(g4.copy(max_tokens=32768), inp, fused=True) == \
        "split_i8_kernel<128,8,2,true,4,true,true,false>"
    assert kvb.batch_kernel_name(g4.copy(batch=1, max_tokens=65536), inp) == "split_i8_kernel<128,8,2,true,4,false,true,false>"
    small_pages = s.copy(page_tokens=16, pages=8192 * 4, table_entries=8192 * 4)
    assert kvb.batch_kernel_name(small_pages, inp).startswith("split_generic_kernel<true, true>")
    assert kvb.batch_kernel_name(s.copy(batch=0), inp) == ""


def test_synth_batch_layout():
    bc = W.synth_batch(1, 8, 2, 64, 64, [100, 0, 257, 64], seed=1, split_tokens=128)
    assert list(bc.seq_starts) == [0, 100, 100, 357, 421]
    assert list(bc.page_offsets) == [0, 2, 2, 7]
    assert sorted(bc.table.tolist()) == list(range(8))  # every pool page used once
    c = bc.sequence(2)
    assert c.shape.tokens == 257 and len(c.table) == 5 and c.qpos.tolist() == [256]
    assert kvb.batch_shape_error(bc.shape) is None
