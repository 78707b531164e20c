"""Host sanitizer run (CPU): the C ABI and C++ host layer (capi.cpp,
attention_shape.cpp, batch_shape.cpp, attention_api.cpp) built by g++ with
AddressSanitizer + UndefinedBehaviorSanitizer, every finding fatal
(tests/cpp/Makefile capi_reject_asan / api_test_asan), running the host-only
checks: the C-ABI rejections and boundary-value sweep of
tests/cpp/capi_reject_test.cpp, the C++ API checks of tests/cpp/api_test.cpp,
and the reference's own tests/shape_test.cpp on this repository's shape code
(oracle/Makefile, when the reference tree is present) -- the counterpart of
the reference's host ASan/UBSan CTest run.  No device is touched."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def binaries():
    r = subprocess.run(["make", "-s", "-C", CPP, "capi_reject_asan", "api_test_asan"], capture_output=True,
                       text=True, timeout=1200)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return {n: os.path.join(CPP, n) for n in ("capi_reject_asan", "api_test_asan")}


def _run(path):
    r = subprocess.run([path], capture_output=True, text=True, timeout=600, env=ENV)
    assert r.returncode == 0 and "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, \
        r.stdout[-3000:] + r.stderr[-3000:]
    return r.stdout


@pytest.mark.timeout(1500)
def test_c_abi_host_checks_under_asan_ubsan(binaries):
    assert "PASS C ABI host checks" in _run(binaries["capi_reject_asan"])


@pytest.mark.timeout(1500)
def test_cpp_api_host_checks_under_asan_ubsan(binaries):
    assert "PASS C++ API host checks" in _run(binaries["api_test_asan"])


def test_reference_shape_test_under_asan_ubsan():
    path = os.path.join(ROOT, "oracle", "_ref", "shape_test_on_repo_asan")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    assert "PASS" in _run(path)


def test_sanitizers_are_live(tmp_path):
    # Planted mistakes under the same flags: a heap read past the end and a
    # signed overflow must each end the program with a sanitizer report (the
    # read may be caught by UBSan's object-size check before ASan's).
    for name, body, tags in [
        ("oob", "int main(int c, char**) { int* p = new int[4]; int v = p[c + 3]; delete[] p; return v; }",
         ("AddressSanitizer", "runtime error")),
        ("ovf", "#include <climits>\nint main(int c, char**) { int x = INT_MAX - 1 + c; return x + c > 0; }",
         ("runtime error",)),
    ]:
        src, exe = tmp_path / f"{name}.cpp", tmp_path / name
        src.write_text(body + "\n")
        r = subprocess.run(["g++", *SAN, str(src), "-o", str(exe)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        r = subprocess.run([str(exe)], capture_output=True, text=True, env=ENV)
        assert r.returncode != 0 and any(t in r.stderr for t in tags), (name, r.returncode, r.stderr[-500:])
