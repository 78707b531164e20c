"""The boundary on a device: the three preload entry points through the C ABI
and through the C++ API (reference src/attention_shared.cu:376-387,
src/attention_mma.cu:13-31) return hipSuccess, and the C++ API's
launch_attention gives the exact result of a one-token cache
(tests/cpp/api_test.cpp --gpu, built by __graft_entry__.build())."""
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
