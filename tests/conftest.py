import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def coracle():
    from oracle import coracle as C
    C.lib()
    return C


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from gemma4metal_amd import turboquant as tq
    return tq


@pytest.fixture
def tq_env():
    """set(name, value) sets a TQ_* kernel-choice switch and makes the
    library re-read its switches; teardown restores the environment and
    re-reads them again."""
    from gemma4metal_amd import turboquant as tq
    saved = {}

    def set_(name, value):
        if name not in saved:
            saved[name] = os.environ.get(name)
        os.environ[name] = str(value)
        tq.reload_options()

    yield set_
    for name, old in saved.items():
        if old is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = old
    if saved:
        tq.reload_options()
