import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    o.set_threads(min(8, os.cpu_count() or 1))
    return o


@pytest.fixture(scope="session")
def dev():
    """A library context on GPU 0 (h3s_open)."""
    from sycl_minimax_h3_amd import Device

    d = Device.open()
    yield d
    d.close()


@pytest.fixture(scope="session")
def dev_wave():
    """A context whose row quantizer takes the one-wavefront-a-row layout at every size (H3S_QUANT_WAVE_MIN_ROWS=0)
    where the row shape allows it, so small parity cases reach the layout long inputs use."""
    from sycl_minimax_h3_amd import Device

    old = os.environ.get("H3S_QUANT_WAVE_MIN_ROWS")
    os.environ["H3S_QUANT_WAVE_MIN_ROWS"] = "0"
    try:
        d = Device.open()
    finally:
        if old is None:
            del os.environ["H3S_QUANT_WAVE_MIN_ROWS"]
        else:
            os.environ["H3S_QUANT_WAVE_MIN_ROWS"] = old
    yield d
    d.close()


@pytest.fixture(scope="session")
def dev_cus16():
    """A context that sizes its grids for 16 compute units (H3S_CUS=16): GEMMs of a few dozen tiles then make whole
    rounds of tiles (XCD renumbering and tile groups, no split along K) at sizes the oracle checks quickly."""
    from sycl_minimax_h3_amd import Device

    old = os.environ.get("H3S_CUS")
    os.environ["H3S_CUS"] = "16"
    try:
        d = Device.open()
    finally:
        if old is None:
            del os.environ["H3S_CUS"]
        else:
            os.environ["H3S_CUS"] = old
    yield d
    d.close()
