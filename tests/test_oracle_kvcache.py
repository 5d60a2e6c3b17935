"""The cached MeanFlow restatement equals full recompute (CPU)."""
from __future__ import annotations

import torch

from conftest import cos_stats
from oracle import dit_ref as R
from oracle.kvcache_ref import FMCacheRef


def _setup(seed=0):
    cfg = R.DitConfig(hidden=128, heads=2, ffn=256, n_blocks=2, latent_dim=16, patch=4)
    W = R.weights_for_regime(R.random_dit_weights(cfg, seed), "bf16")
    return cfg, W


def test_cached_solve_equals_full_recompute():
    cfg, W = _setup()
    lens, hist, noise = R.synthetic_requests(1, 30, 30, cfg, seed=3)
    h = hist[0]
    g = R.round_bf16(0.3 * torch.randn(cfg.hidden, generator=torch.Generator().manual_seed(1)))
    full = R.meanflow_solve_varlen(W, cfg, [h], g[None], noise, 4, "bf16")
    cache = FMCacheRef(W, cfg, 4, g, "bf16")
    cache.extend(h[:-1])                       # prefix = rows [0, c-1)
    got = cache.solve(h[-1], noise[0])         # active = last hidden + latents
    assert cos_stats(got, full[0], cfg.latent_dim)[0] > 0.9999


def test_incremental_extend_equals_single_prefill():
    cfg, W = _setup(1)
    lens, hist, noise = R.synthetic_requests(1, 25, 25, cfg, seed=4)
    h = hist[0]
    a = FMCacheRef(W, cfg, 4, None, "bf16")
    a.extend(h[:-1])
    b = FMCacheRef(W, cfg, 4, None, "bf16")
    b.extend(h[:10])
    b.extend(h[10:-1])
    za = a.solve(h[-1], noise[0])
    zb = b.solve(h[-1], noise[0])
    assert cos_stats(za, zb, cfg.latent_dim)[0] > 0.99999
    for k in range(4):
        for l in range(cfg.n_blocks):
            assert torch.allclose(a.kv[k][l][0], b.kv[k][l][0], atol=0.05)
