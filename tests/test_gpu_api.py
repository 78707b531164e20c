"""The boundary on a device: the three preload entry points through the C ABI
and through the C++ API (reference src/attention_shared.cu:376-387,
src/attention_mma.cu:13-31) return hipSuccess, and the C++ API's
launch_attention gives the exact result of a one-token cache
(tests/cpp/api_test.cpp --gpu, built by __graft_entry__.build()); the
diagnostic paged read probe runs on every page size it accepts."""
import os
import subprocess

import pytest

import kvbridge_amd as kvb

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
API_TEST = os.path.join(ROOT, "tests", "cpp", "api_test")


def test_preload_entry_points_return_success(gpu):
    assert kvb.preload_attention_reference_kernels() == 0
    assert kvb.preload_attention_mma_kernels() == 0
    assert kvb.preload_attention_kernels() == 0


def test_cpp_api_on_device(gpu):
    if not os.path.exists(API_TEST):
        pytest.fail(f"{API_TEST} is missing: run __graft_entry__.build() (make -C tests/cpp)")
    r = subprocess.run([API_TEST, "--gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS C++ API device checks" in r.stdout


@pytest.mark.parametrize("dim,page", [(256, 32), (128, 16), (128, 64), (64, 32)])
def test_paged_read_probe_runs(gpu, dim, page):
    """The diagnostic read probe (kvb_paged_read_probe) on 16-, 32- and
    64-token pages, a sequence that ends mid-tile: the launch succeeds and the
    sink (written only if the XOR of everything read hits a fixed value)
    stays zero; pages of other sizes are refused before any launch."""
    import torch
    from kvbridge_amd import workloads as W

    s, t = W.torch_cache(1, 8, 2, dim, page, 1000, seed=7 + dim + page, device="cuda:0")
    inp = kvb.device_input(t["q"], t["qpos"], t["kpos"], t["table"], t["k"], t["v"], t["ks"], t["vs"])
    sink = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    for split_tokens in (256, 1024):
        kvb.paged_read_probe(s, inp, split_tokens, sink)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    s48, t48 = W.torch_cache(1, 8, 2, dim, 48, 1000, seed=3, device="cuda:0")
    inp48 = kvb.device_input(t48["q"], t48["qpos"], t48["kpos"], t48["table"], t48["k"], t48["v"], t48["ks"],
                             t48["vs"])
    with pytest.raises(kvb.KvbInvalidArgument, match="pages of 16, 32 or a multiple of 64"):
        kvb.paged_read_probe(s48, inp48, 256, sink)
