import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fp8-compatibility-layer_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this container")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture
def tune():
    """Sets libtfp8_hip.so tuning knobs for one test (tune(TFP8_GEMM_SPLITK=3, ...)); every knob is
    back at its load-time value afterwards."""
    from tfp8 import _ext

    def set_knobs(**knobs):
        for k, v in knobs.items():
            _ext.tuning_set(k, int(v))
    yield set_knobs
    _ext.tuning_reset()
