import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "smel-ft_amd")
for p in (ROOT, PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C-ABI library)")


@pytest.fixture(scope="session")
def golden_c1():
    from safetensors.torch import load_file
    return load_file(os.path.join(GOLDEN, "c1_moe_fp32.safetensors"))


@pytest.fixture(scope="session")
def golden_quant():
    from safetensors.torch import load_file
    return load_file(os.path.join(GOLDEN, "quant_int4.safetensors"))
