import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def progress(pytestconfig):
    """print() that reaches the terminal past pytest's output capture, so a
    test that runs for minutes shows it is alive to a runner that stops
    silent jobs."""
    capman = pytestconfig.pluginmanager.getplugin("capturemanager")

    def say(*args):
        with capman.global_and_fixture_disabled():
            print(*args, flush=True)
    return say


@pytest.fixture(scope="session")
def lib():
    from qwen35_amd import abi
    return abi.load()
