"""The drop-in boundary without a GPU: every function declared in
include/kvbridge_c.h is exported by libkvbridge_amd.so and bound in
kvbridge_amd/_capi.py; the headers compile; the C++ API keeps the
reference's exception types and messages; and the reference's own host
tests (tests/shape_test.cpp, tests/reference_test.cpp), compiled against this
repository's headers and sources by oracle/Makefile, pass."""
import os
import re
import subprocess

import pytest

import kvbridge_amd as kvb
from kvbridge_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C_HEADER = os.path.join(ROOT, "include", "kvbridge_c.h")
REF_BIN = os.path.join(ROOT, "oracle", "_ref")


def declared_functions():
    text = open(C_HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kvb_\w+)\s*\(", text))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("kvb_shape_error", "kvb_split_count", "kvb_scratch_elements", "kvb_launch_attention",
                 "kvb_launch_attention_mma", "kvb_merge_attention", "kvb_preload_attention_kernels",
                 "kvb_split_attention", "kvb_merge_finalize", "kvb_decode_attention"):
        assert must in names


def test_every_declared_symbol_is_exported_and_bound():
    lib = kvb.load()
    bound = {name for name, _, _ in _capi.SIGNATURES}
    declared = declared_functions()
    assert declared == bound, (declared ^ bound)
    for name in declared:
        assert hasattr(lib, name), name


def test_c_header_is_plain_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "kvbridge_c.h"\nint main(void) { kvb_shape s = {0}; return kvb_shape_valid(&s); }\n')
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_api_exceptions(tmp_path):
    exe = tmp_path / "api_test"
    r = subprocess.run(["hipcc", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "cpp", "api_test.cpp"), "-L", os.path.join(ROOT, "kvbridge_amd"),
                        "-lkvbridge_amd", f"-Wl,-rpath,{os.path.join(ROOT, 'kvbridge_amd')}", "-o", str(exe)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout


@pytest.mark.parametrize("binary,expect", [
    ("shape_test_on_repo", "PASS"),          # reference shape KATs on this repo's shape code
    ("reference_test_on_repo", "oracle checks passed"),
    ("ref_shape_test", "PASS"),              # the same tests on the reference's own code
    ("ref_reference_test", "oracle checks passed"),
])
def test_reference_host_tests(binary, expect):
    path = os.path.join(REF_BIN, binary)
    if not os.path.exists(path):
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    r = subprocess.run([path], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert expect in r.stdout


def test_kernel_choice_for_the_dense_mma_geometry():
    """rows 8 / group 6 / dim 256 / page 32 (the reference's MMA geometry): 48
    head-rows in 3 blocks of 16.  Splits that start on a 64-token tile run the
    int8-MFMA rows kernel, which streams each split's KV once for every
    head-row block; an off-tile start runs the per-block LDS kernel.
    KVB_SPLIT_IMPL=f16 would pick the f16 kernels."""
    fake = 0x1000
    inp = kvb.device_input(fake, fake, fake, fake, fake, fake, fake, fake)
    s = kvb.make_shape(8, 24, 4, 256, 32, 2048, 65536, 0, 65536, 0.0625)
    assert kvb.attention_mma_supported(s)
    assert kvb.selected_kernel_name(s, inp, 256) == "split_i8_rows_pc_kernel<256,false>"
    assert kvb.selected_kernel_name(s, inp, 1024) == "split_i8_rows_pc_kernel<256,false>"
    assert kvb.selected_kernel_name(s, inp, 1000).startswith("split_lds_kernel<256,")  # off-tile split size
    assert kvb.selected_kernel_name(s.copy(begin=32), inp, 256).startswith("split_lds_kernel<256,")  # off-tile start
    s128 = kvb.make_shape(8, 48, 8, 128, 64, 10, 640, 64, 640, 0.0883883)
    assert kvb.selected_kernel_name(s128, inp, 256) == "split_i8_rows_kernel<128,true>"
    s64 = kvb.make_shape(8, 48, 8, 64, 64, 10, 640, 64, 640, 0.125)
    assert kvb.selected_kernel_name(s64, inp, 256).startswith("split_lds_rows_kernel<64,")  # dim 64: f16 rows kernel
