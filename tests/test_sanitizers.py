"""The oracle and the C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

Each check runs other CPU test files in a child pytest with a sanitizer runtime preloaded and the
fixtures pointed at sanitized builds (tests/conftest.py):

- the oracle (oracle/liboracle_san_l8.so, liboracle_san_l16.so: gcc, -fsanitize=address,undefined)
  under the oracle and checkpoint tests;
- libtsfm_attn with its host code sanitized (tsfm-zig_amd/_build/san/libtsfm_attn_san.so: the
  ABI's .cpp files built with -fsanitize on the host pass, the device code as shipped) under the ABI
  tests, including the validation fuzz.

Without a GPU the ABI runs its validation, bookkeeping and error paths, not the staging around a
launch. Any sanitizer report fails the child (halt on the first error).
"""
import glob
import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def preload_free():
    # The sanitizer runtime must be the first library the child loads; a preload configured by
    # the environment is left as it is, and the check is skipped.
    if os.environ.get("LD_PRELOAD"):
        pytest.skip("LD_PRELOAD is already set; the sanitizer runtime has to load first")


def _gcc_asan():
    p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not p or not os.path.exists(p):
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    return p


def _clang_asan():
    libs = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not libs:
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    return libs[-1]


def _child(preload, extra_env, files):
    env = dict(os.environ, LD_PRELOAD=preload, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", **extra_env)
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *files],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out, out[-2000:]


def test_oracle_under_sanitizers(preload_free):
    rt = _gcc_asan()
    subprocess.run(["make", "-C", str(ROOT / "oracle"), "liboracle_san_l8.so", "liboracle_san_l16.so"], check=True,
                   capture_output=True)
    _child(rt, {"TSFM_TEST_ORACLE_SANITIZED": "1"}, ["tests/test_oracle.py", "tests/test_checkpoint.py"])


def test_abi_host_code_under_sanitizers(preload_free):
    rt = _clang_asan()
    r = subprocess.run(["make", "-C", str(ROOT / "tsfm-zig_amd"), "sanitize"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    lib = ROOT / "tsfm-zig_amd" / "_build" / "san" / "libtsfm_attn_san.so"
    _child(rt, {"TSFM_TEST_PRODUCT_LIB": str(lib)}, ["tests/test_abi.py"])
