"""Cached MeanFlow solve (prefix K/V cache) vs full recompute. GPU only.
Tolerance as the full solve: per-row cosine >= 0.9999, max |diff| <= 2% of max |ref|,
against the oracle's full-recompute solve in both regimes (fp32: the
fixture-pinned parity bar; bf16: the autocast restatement)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import cos_stats
from oracle import dit_ref as R
from oracle.kvcache_ref import FMCacheRef
from test_gpu_parity import _assert_vs_fp32

pytestmark = pytest.mark.gpu

CFG = R.DitConfig(hidden=256, heads=4, ffn=1024, n_blocks=2, latent_dim=64, patch=16)


def _head(cfg, seed):
    from nanovllm_dots_amd import FMSpec, HipFMHead
    W = R.random_dit_weights(cfg, seed)
    return HipFMHead(FMSpec.of(cfg), W, device="cuda"), R.weights_for_regime(W, "bf16")


def _pad(rows_list, H):
    m = max(1, max(r.shape[0] for r in rows_list))
    out = torch.zeros(len(rows_list), m, H)
    for i, r in enumerate(rows_list):
        out[i, :r.shape[0]] = r
    return out


def _check(got, ref, ld, label):
    got, ref = got.float().cpu(), ref.float().cpu()
    cmin, _ = cos_stats(got, ref, ld)
    err = (got - ref).abs().max().item()
    print(f"{label}: cos min {cmin:.6f} maxabs {err:.4g}", flush=True)
    assert cmin >= 0.9999 and err <= 0.02 * ref.abs().max().item()


def test_cached_solve_matches_full_recompute_oracle():
    from nanovllm_dots_amd import HipFMCache
    head, Wb = _head(CFG, 5)
    lens, hist, noise = R.synthetic_requests(3, 20, 300, CFG, seed=7)
    g = R.round_bf16(torch.from_numpy(0.3 * np.random.RandomState(2).standard_normal((3, CFG.hidden)).astype(np.float32)))
    ref = R.meanflow_solve_varlen(Wb, CFG, hist, g, noise, 4, "bf16")
    cache = HipFMCache(head, 3, max(lens) + 32, 4)
    prefix = [h[:-1] for h in hist]
    cache.extend(_pad(prefix, CFG.hidden).cuda(), [p.shape[0] for p in prefix], g_cond=g.cuda())
    assert cache.lengths == [L - 1 for L in lens]
    lh = torch.stack([h[-1] for h in hist]).cuda()
    got = cache.solve(lh, g_cond=g.cuda(), noise=noise.cuda())
    _check(got, ref, CFG.latent_dim, "cached-vs-full")
    _assert_vs_fp32(got, Wb, CFG, hist, g, noise, "cached")


def test_cached_solve_matches_cached_oracle_and_incremental_extend():
    from nanovllm_dots_amd import HipFMCache
    head, Wb = _head(CFG, 6)
    lens, hist, noise = R.synthetic_requests(2, 60, 140, CFG, seed=9)
    cache = HipFMCache(head, 2, 200, 4)
    split = [h.shape[0] // 3 for h in hist]
    first = [h[:s] for h, s in zip(hist, split)]
    second = [h[s:-1] for h, s in zip(hist, split)]
    cache.extend(_pad(first, CFG.hidden).cuda(), [r.shape[0] for r in first])
    cache.extend(_pad(second, CFG.hidden).cuda(), [r.shape[0] for r in second])
    lh = torch.stack([h[-1] for h in hist]).cuda()
    got = cache.solve(lh, noise=noise.cuda())
    for i in range(2):
        ref_cache = FMCacheRef(Wb, CFG, 4, None, "bf16")
        ref_cache.extend(hist[i][:-1])
        ref = ref_cache.solve(hist[i][-1], noise[i])
        _check(got[i], ref, CFG.latent_dim, f"cached-oracle stream {i}")


def test_cached_matches_direct_hip_solve():
    """The cached solve and the direct solve of the same sequences agree."""
    from nanovllm_dots_amd import HipFMCache, HipMeanflow
    head, _ = _head(CFG, 8)
    lens, hist, noise = R.synthetic_requests(4, 5, 260, CFG, seed=11)
    inp, mask, pos, g = R.pack_fm_inputs(hist, CFG.patch, CFG.hidden)
    bf = lambda t: t.to("cuda", torch.bfloat16)
    direct = HipMeanflow(None, num_steps=4, dit=object(), head=head)(
        input_sequence=bf(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=bf(g), noise=bf(noise))
    cache = HipFMCache(head, 4, max(lens) + 24, 4)
    prefix = [h[:-1] for h in hist]
    cache.extend(_pad(prefix, CFG.hidden).cuda(), [p.shape[0] for p in prefix])
    got = cache.solve(torch.stack([h[-1] for h in hist]).cuda(), noise=bf(noise))
    _check(got, direct, CFG.latent_dim, "cached-vs-direct")


def test_capacity_overflow_raises():
    from nanovllm_dots_amd import HipFMCache
    head, _ = _head(CFG, 1)
    cache = HipFMCache(head, 1, 40, 4)
    with pytest.raises(RuntimeError, match="capacity"):
        cache.extend(torch.zeros(1, 30, CFG.hidden).cuda(), [30])
    cache.extend(torch.zeros(1, 20, CFG.hidden).cuda(), [20])
    assert cache.lengths == [20]


def test_full_size_long_prefix():
    """12 blocks, H=1024; two streams with 2,000-row prefixes, cached vs oracle full recompute."""
    from nanovllm_dots_amd import HipFMCache
    cfg = R.DitConfig(hidden=1024, heads=16, ffn=4096, n_blocks=12, latent_dim=64, patch=16)
    head, Wb = _head(cfg, 2)
    lens, hist, noise = R.synthetic_requests(2, 2000, 2000, cfg, seed=12)
    ref = R.meanflow_solve_varlen(Wb, cfg, hist, None, noise, 4, "bf16")
    cache = HipFMCache(head, 2, 2048, 4)
    prefix = [h[:-1] for h in hist]
    cache.extend(_pad(prefix, cfg.hidden).cuda(), [p.shape[0] for p in prefix])
    got = cache.solve(torch.stack([h[-1] for h in hist]).cuda(), noise=noise.cuda())
    _check(got, ref, cfg.latent_dim, "full-size cached")
    _assert_vs_fp32(got, Wb, cfg, hist, None, noise, "full-size cached", device="cuda")


@pytest.mark.parametrize("path", ["direct", "cached"])
def test_ksplit_matches_whole_tiles(path):
    """The K-split of the last partial round of GEMM tiles against whole tiles
    (float32 partial sums in piece order: agreement to bf16 rounding)."""
    from nanovllm_dots_amd import HipFMCache, HipMeanflow
    head, _ = _head(CFG, 8)
    lens, hist, noise = R.synthetic_requests(4, 5, 260, CFG, seed=11)
    bf = lambda t: t.to("cuda", torch.bfloat16)
    outs = []
    for ks in (False, True):
        head.set_ksplit(ks)
        if path == "direct":
            inp, mask, pos, g = R.pack_fm_inputs(hist, CFG.patch, CFG.hidden)
            out = HipMeanflow(None, num_steps=4, dit=object(), head=head)(
                input_sequence=bf(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=bf(g), noise=bf(noise))
        else:
            cache = HipFMCache(head, 4, max(lens) + 24, 4)
            prefix = [h[:-1] for h in hist]
            cache.extend(_pad(prefix, CFG.hidden).cuda(), [p.shape[0] for p in prefix])
            out = cache.solve(torch.stack([h[-1] for h in hist]).cuda(), noise=bf(noise))
        outs.append(out)
    head.set_ksplit(True)
    _check(outs[1], outs[0], CFG.latent_dim, f"ksplit-vs-whole {path}")


def test_decode_chunks_ragged_streams_and_repeated_solves():
    """Streams whose prefixes span one to 13 key chunks in one launch (a stream
    of one chunk writes its rows directly, the others merge their chunk
    partials in the last chunk to finish), a group count (3 streams x 4 heads)
    that is not a multiple of 8, and solves repeated on the same cache: the
    merge counters return to zero and the chunk-order merge repeats bit for bit."""
    from nanovllm_dots_amd import HipFMCache
    head, Wb = _head(CFG, 3)
    rs = np.random.RandomState(21)
    hist = [R.round_bf16(torch.from_numpy((0.5 * rs.standard_normal((n, CFG.hidden))).astype(np.float32)))
            for n in (41, 1500, 3101)]
    noise = R.round_bf16(torch.from_numpy(rs.standard_normal((3, CFG.patch, CFG.latent_dim)).astype(np.float32)))
    ref = R.meanflow_solve_varlen(Wb, CFG, hist, None, noise, 4, "bf16")
    cache = HipFMCache(head, 3, 3136, 4)
    prefix = [h[:-1] for h in hist]
    cache.extend(_pad(prefix, CFG.hidden).cuda(), [p.shape[0] for p in prefix])
    lh = torch.stack([h[-1] for h in hist]).cuda()
    first = cache.solve(lh, noise=noise.cuda())
    _check(first, ref, CFG.latent_dim, "ragged cached")
    for rep in range(2):
        again = cache.solve(lh, noise=noise.cuda())
        assert torch.equal(again, first), f"repeat {rep}"


def test_many_back_to_back_extends():
    """Twelve extends in a row with no host wait between them (their uploads
    cycle through the ring of pinned staging slots and reuse them) agree with
    one extend of the same rows."""
    from nanovllm_dots_amd import HipFMCache
    head, _ = _head(CFG, 4)
    lens, hist, noise = R.synthetic_requests(2, 150, 200, CFG, seed=13)
    prefix = [h[:-1] for h in hist]
    lh = torch.stack([h[-1] for h in hist]).cuda()
    whole = HipFMCache(head, 2, 256, 4)
    whole.extend(_pad(prefix, CFG.hidden).cuda(), [p.shape[0] for p in prefix])
    ref = whole.solve(lh, noise=noise.cuda())
    inc = HipFMCache(head, 2, 256, 4)
    cuts = [np.linspace(0, p.shape[0], 13).astype(int) for p in prefix]
    for k in range(12):
        parts = [p[c[k]:c[k + 1]] for p, c in zip(prefix, cuts)]
        inc.extend(_pad(parts, CFG.hidden).cuda(), [q.shape[0] for q in parts])
    assert inc.lengths == [p.shape[0] for p in prefix]
    got = inc.solve(lh, noise=noise.cuda())
    _check(got, ref, CFG.latent_dim, "12 extends vs one")
