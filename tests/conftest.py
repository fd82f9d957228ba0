"""Shared pytest setup: import paths, the `gpu` marker, device fixtures."""
from __future__ import annotations

import pytest

from tests import helpers  # noqa: F401  (puts the repo root and package dir on sys.path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; fails loudly (not skips) when absent."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but torch.cuda.is_available() is False")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def llmik(cuda):
    import llmik_cuda
    return llmik_cuda
