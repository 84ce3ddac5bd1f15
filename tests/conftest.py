"""Shared pytest setup: the `gpu` marker and import paths.

The package directory `universal-lm-trainer_amd/` holds the drop-in module
`flash_attn_v100_cuda` (the reference's module name) and is put on sys.path the
way train.py puts its own directory there; the repo root is added for `oracle`.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "universal-lm-trainer_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def gpu_available():
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def fa():
    """The drop-in module with its extension loaded; a GPU test fails loudly
    (never skips) when the native extension did not load."""
    import flash_attn_v100_cuda as mod
    assert mod.is_available(), f"native extension not loaded: {mod.build_error()}"
    return mod
