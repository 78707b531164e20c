"""a five-layer decode step.  Five independent layers,
each with its own paged INT8 KV cache at the cfg2 shape (32q/8kv heads,
head_dim 128, 65536 tokens, page 64, random page tables, per-(token, kv
head) scales), each doing split-K partials plus merge through the
single-launch call, run back to back on one stream and captured once in a
HIP graph.  Every replay must equal the eager step bitwise, and every
layer's output must pass the north-star gate against the FP64 oracle."""
import numpy as np
import pytest

import kvbridge_amd as kvb
from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import log

pytestmark = pytest.mark.gpu

LAYERS = 5
SPLIT_TOKENS = 2048


def test_five_layer_graph_step(gpu):
    import torch

    layers = []
    for i in range(LAYERS):
        shape, t = W.torch_cache(1, 32, 8, 128, 64, 65536, seed=0x4B56425 + i, device="cuda:0")
        inp = kvb.device_input(t["q"], t["qpos"], t["kpos"], t["table"], t["k"], t["v"], t["ks"], t["vs"])
        layers.append(dict(
            shape=shape, t=t, inp=inp,
            scratch=torch.empty(kvb.scratch_elements(shape, SPLIT_TOKENS), dtype=torch.float32, device=gpu),
            counters=torch.zeros(shape.kv_heads, dtype=torch.int32, device=gpu),
            m=torch.empty(32, dtype=torch.float32, device=gpu), l=torch.empty(32, dtype=torch.float32, device=gpu),
            n=torch.empty(32 * 128, dtype=torch.float32, device=gpu),
            out=torch.zeros(32 * 128, dtype=torch.float16, device=gpu)))
    log(f"five-layer step: kernel={kvb.selected_kernel_name(layers[0]['shape'], layers[0]['inp'], SPLIT_TOKENS, True)}")
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()  # the caches were generated on the default stream

    def step():
        for L in layers:
            kvb.decode_attention_fused(L["shape"], L["inp"], SPLIT_TOKENS, L["scratch"], L["counters"], L["m"],
                                       L["l"], L["n"], L["out"], kvb.KVB_OUT_F16, stream.cuda_stream)

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    eager = [L["out"].clone() for L in layers]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    for rep in range(3):
        for L in layers:
            L["out"].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, L in enumerate(layers):
            assert torch.equal(L["out"], eager[i]), f"replay {rep}: layer {i} differs from eager"
            assert torch.count_nonzero(L["counters"]).item() == 0
    log(f"  3 graph replays of the {LAYERS}-layer step equal the eager step")
    for i, L in enumerate(layers):
        t = L["t"]
        case = W.Case(L["shape"], t["q"].cpu().numpy(), t["qpos"].cpu().numpy(), t["kpos"].cpu().numpy(),
                      t["table"].cpu().numpy().view(np.uint32), t["k"].cpu().numpy(), t["v"].cpu().numpy(),
                      t["ks"].cpu().numpy(), t["vs"].cpu().numpy())
        ref, vis = O.fp64(case, threads=16)
        assert vis.all()
        gate = O.gates(eager[i].float().cpu().numpy().reshape(32, 128), ref)
        log(f"  layer {i}: max_abs={gate['max_abs']:.2e} rel_l2={gate['rel_l2']:.2e}")
        assert gate["pass"], gate
