import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def _has_gpu() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    if not _has_gpu():
        pytest.skip("no HIP device")
    import torch

    return torch.device("cuda:0")


@pytest.fixture
def tuning():
    """Sets libdaser_kv launch-shape overrides (dsr_set_tuning) for one
    test and restores every knob it touched to the default afterwards."""
    from daser_amd import _lib

    touched = set()

    def set_knob(knob, value):
        touched.add(knob)
        _lib.set_tuning(knob, value)

    yield set_knob
    for knob in touched:
        _lib.set_tuning(knob, 0)
