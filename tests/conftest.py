"""Shared test set-up: repo root on sys.path, the `gpu` marker, CPU threads."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _few_cpu_threads():
    import torch
    old = torch.get_num_threads()
    torch.set_num_threads(min(4, old))
    yield
    torch.set_num_threads(old)


@pytest.fixture(scope="session")
def host_runner(tmp_path_factory):
    """The AddressSanitizer host build of the kernels (tests/host_emu/), built
    once per session and shared by the emulated-kernel tests."""
    from tests.host_emu import harness
    if harness.compiler() is None:
        pytest.skip("no host clang")
    return harness.build(str(tmp_path_factory.mktemp("host_emu")))
