"""Shared pytest setup: the `gpu` marker and import paths.

Tests marked `gpu` need a HIP device (an MI355X on the GPU box); everything
else runs on the CPU container.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "kraken-infer_amd", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X)")


@pytest.fixture(scope="session")
def hip_ctx():
    """One HIP context for the whole GPU session (skips cleanly on CPU).

    torch (which carries its own HIP runtime) is initialised first when it sees
    the GPU, as bench.py does, so that tests can hand torch streams and graph
    captures to the library."""
    try:
        import torch

        if torch.cuda.is_available():
            torch.cuda.init()
    except ImportError:
        pass
    import kraken_hip

    ctx = kraken_hip.Context()
    yield ctx
    ctx.close()
