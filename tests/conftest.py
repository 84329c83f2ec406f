"""pytest configuration: the `gpu` marker, import paths, and the built libraries."""
import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "tsfm-zig_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) GPU")


# A sanitizer run (tests/test_sanitizers.py) points the oracle fixtures at the ASan/UBSan builds
# (liboracle_san_l8.so / liboracle_san_l16.so) and the product fixture at the sanitized library
# through these variables.
ORACLE_SANITIZED = os.environ.get("TSFM_TEST_ORACLE_SANITIZED") == "1"
PRODUCT_OVERRIDE = os.environ.get("TSFM_TEST_PRODUCT_LIB")


def _ensure_oracle():
    """The oracle is plain C; build it here if build() has not run yet (gcc only)."""
    lib = ROOT / "oracle" / "liboracle_l8.so"
    if not lib.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)


def _oracle_lib(name):
    return ROOT / "oracle" / (name.replace("liboracle_", "liboracle_san_") if ORACLE_SANITIZED else name)


@pytest.fixture(scope="session")
def orc():
    _ensure_oracle()
    import _oracle

    return _oracle.Oracle(_oracle_lib("liboracle_l8.so"))


@pytest.fixture(scope="session")
def orc16():
    _ensure_oracle()
    import _oracle

    return _oracle.Oracle(_oracle_lib("liboracle_l16.so"))


def host_has_avx512() -> bool:
    info = pathlib.Path("/proc/cpuinfo")
    return info.exists() and " avx512f" in info.read_text()


@pytest.fixture(scope="session")
def orc_host():
    """The oracle with the f32 lane count the reference would use on this host (nn.lanes =
    suggestVectorLength(f32), src/core/nn.zig:296): 16 on AVX-512, else 8."""
    _ensure_oracle()
    import _oracle

    return _oracle.Oracle(_oracle_lib("liboracle_l16.so" if host_has_avx512() else "liboracle_l8.so"))


@pytest.fixture(scope="session")
def ta():
    """The product binding (tsfm-zig_amd/tsfm_attn); fails if the library is not built."""
    import tsfm_attn

    if PRODUCT_OVERRIDE:
        tsfm_attn._lib = tsfm_attn.load(PRODUCT_OVERRIDE)
    else:
        tsfm_attn.load()
    return tsfm_attn


@pytest.fixture(scope="session")
def gpu_ready(ta):
    """For gpu tests: the library must see a gfx950 device; anything else is a failure, not a skip."""
    if os.environ.get("TSFM_HIP_DISABLE"):
        pytest.fail("TSFM_HIP_DISABLE is set in a gpu test run")
    if not ta.available():
        pytest.fail(f"libtsfm_attn sees no usable gfx950 device: {ta.last_error()}")
    import torch

    assert torch.cuda.is_available()
    return True
