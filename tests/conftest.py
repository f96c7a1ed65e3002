"""pytest setup: the `gpu` marker, import paths for the package and the oracle."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "ggml-compiler_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libgcq.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gops():
    """libgcq's ops on cuda:0. No skip: on a GPU run a missing library or device is a failure."""
    import torch  # noqa: F401

    from ggml_compiler_amd import ops

    ops.require_device()
    return ops


def to_np(t):
    return t.detach().cpu().numpy()
