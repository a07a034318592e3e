"""Shared fixtures and markers.

Tests marked `gpu` need an MI355X (gfx950) and the built libkf950.so; everything else
runs on the CPU. A GPU test never falls back to a PyTorch path: it calls the native
kernels (directly, or through FusedTransformer with KF950_STRICT=1) and fails if they are
not there.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import torch  # noqa: E402


def _has_gpu() -> bool:
    try:
        return torch.cuda.is_available() and torch.cuda.device_count() > 0
    except Exception:
        return False


HAS_GPU = _has_gpu()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libkf950.so")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    return torch.device("cuda" if HAS_GPU else "cpu")


@pytest.fixture(autouse=True)
def _strict_native(monkeypatch):
    """The drop-in re-raises instead of falling back, so a native failure is visible."""
    monkeypatch.setenv("KF950_STRICT", "1")


def make_model(cfg, seed: int = 7, random_norms: bool = False, device="cpu"):
    from techjam2026_amd import harness
    from techjam2026_amd.model import BaselineTransformer
    model = BaselineTransformer(cfg)
    harness.init_weights_(model, seed, random_norms=random_norms)
    return model.to(device).eval()


def params_of(model):
    return {k: v.detach().cpu() for k, v in model.state_dict().items()}
