"""Shared fixtures. `gpu`-marked tests need an MI355X; everything else runs on
the CPU (oracle pinning, host logic, ABI loading)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from shady_thinker_amd import GpuContext

    ctx = GpuContext(0)
    yield ctx
    ctx.close()


@pytest.fixture
def tune(gpu):
    """tune(KNOB=value, ...): force kernel-path settings of the shared context
    (st_context_set_tune) for the rest of the test; all restored after it."""
    from shady_thinker_amd._lib import TUNE_KNOBS

    saved = {k: gpu.get_tune(k) for k in TUNE_KNOBS}

    def set_(**knobs):
        for k, v in knobs.items():
            gpu.set_tune(k, int(v))

    yield set_
    for k, v in saved.items():
        gpu.set_tune(k, v)
