import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libmimizuku_amd.so")


def has_gpu() -> bool:
    return os.path.exists("/dev/kfd")


def pytest_collection_modifyitems(config, items):
    if has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU (/dev/kfd absent)")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def large_v3_weights():
    """Seeded random-init weights of the full large-v3 geometry (1.5 G parameters, fp16), drawn once per session for
    the GPU tests that run the whole model."""
    from mimizuku_amd import synth
    return synth.random_weights(synth.LARGE_V3, seed=8, bias_std=0.02, ln_std=0.1)
