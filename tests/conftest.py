"""pytest configuration: the `gpu` marker, import paths, and shared helpers.

`-m "not gpu"` runs the oracle pins, the stored-form conversions, the host refusals and the library's exported
symbols on the CPU; `-m gpu` runs the parity tests proper, through the C-ABI, on a real MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "radiance-exl3_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) and the built libexl3c4.so")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ref_common():
    """The REFERENCE's own common/exl3_decode.c + exl3_layout.c, compiled by oracle/Makefile into oracle/_ref (only
    where /root/reference exists: this container; the GPU box has no reference)."""
    import ctypes
    import oracle
    if not os.path.exists(oracle.REF_PATH):
        if os.path.isdir("/root/reference/common"):
            oracle.build(ref=True)
    if not os.path.exists(oracle.REF_PATH):
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return ctypes.CDLL(oracle.REF_PATH)
