"""Shared test setup: the ``gpu`` marker, repo import path, cosine helpers."""
from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    has_gpu = torch.cuda.is_available()
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords and not has_gpu:
            it.add_marker(skip)


def cos_stats(a, b, latent_dim=None):
    """Per-row cosine similarity -> (min, mean) (rows of ``latent_dim`` when given)."""
    a, b = a.float(), b.float()
    if latent_dim is not None:
        a, b = a.reshape(-1, latent_dim), b.reshape(-1, latent_dim)
    c = torch.nn.functional.cosine_similarity(a, b, dim=-1)
    return c.min().item(), c.mean().item()


def load_golden(name):
    import numpy as np
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))
