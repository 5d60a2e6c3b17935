"""The benchmark configurations on the GPU, at their own sizes. GPU only.

* One DiT block (hidden 1024, 16 x 64 heads, MLP 4096), 64 context + 16
  latent rows, t = dt = 0.25, seed 0: the HIP forward against the output that
  the reference's own float32 DiT wrote into tests/golden/c1_block.npz (float32
  weights there; the HIP head holds them in bf16). Bar: per-row cosine >= 0.9999
  and max |diff| <= 0.01 * max |ref| over all 80 rows.
* The 64-request batch exactly as bench.py builds it (64 requests, contexts
  U{64..1024}, seed 0, 12 blocks): one HIP solve of all 64; four requests (the
  longest, 1024 rows; the second longest; the shortest; request 0) against the
  fp32 oracle's solve of each request alone (requests are independent: padding
  transparency). Bar: the solve's, cosine >= 0.9999 and max |diff| <=
  0.02 * max |ref|.
* The long-audio cache as bench.py builds it (512 context + 600 x 16 patch
  rows = 10,112 rows per stream, the last one the active hidden row): one stream
  cached against the fp32 oracle's full recompute of all 10,112 + 16 rows (run
  with torch's float32 kernels on the GPU; 12 TFLOP is too much for the host);
  then the 4-stream cache against each stream cached alone.
* The W8A8 GEMM's int32 accumulators of the W8A8 GEMM bit-exact against torch._int_mm at
  M = 8192 and 16384 for the four (K, N) shapes.
"""
from __future__ import annotations

import ast

import numpy as np
import pytest
import torch

from conftest import cos_stats, load_golden
from oracle import dit_ref as R
from test_gpu_parity import FULL, LAT_COS, _assert_latents, _cuda_bf16, _fp32_solve

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_head():
    """The bench's 12-block head (seed-0 weights) and its bf16-valued parameters."""
    from nanovllm_dots_amd import FMSpec, HipFMHead
    W = R.random_dit_weights(FULL, 0)
    head = HipFMHead(FMSpec.of(FULL), W, device="cuda")
    yield head, R.weights_for_regime(W, "bf16")
    head.close()


def test_one_block_80_rows_matches_reference_fixture():
    from nanovllm_dots_amd import FMSpec, HipDiT, HipFMHead
    g = load_golden("c1_block.npz")
    cfg = R.DitConfig(**ast.literal_eval(str(g["cfg"])))
    assert cfg.n_blocks == 1 and cfg.hidden == 1024
    head = HipFMHead(FMSpec.of(cfg), R.random_dit_weights(cfg, 0), device="cuda")
    rs = np.random.RandomState(0)
    x = torch.from_numpy(rs.standard_normal((1, 80, 1024)).astype(np.float32))
    pos = R.build_fm_pos_ids(64, 80, 16)[None]
    t = torch.full((1,), 0.25)
    print("one block: 1 x (64 + 16) rows, t = dt = 0.25", flush=True)
    got = HipDiT(head=head, strict=True)(x=_cuda_bf16(x), timesteps=t.cuda(), duration=t.cuda(),
                                         pos_ids=pos.cuda(), g_cond=torch.zeros(1, 1024, device="cuda",
                                                                                dtype=torch.bfloat16))
    got = got.float().cpu()[0]
    ref = torch.from_numpy(g["out"])[0]
    cmin, cmean = cos_stats(got, ref)
    err = (got - ref).abs().max().item()
    print(f"one block vs reference fixture: cos min {cmin:.6f} mean {cmean:.6f} maxabs {err:.4g} "
          f"(|ref| {ref.abs().max().item():.3g})", flush=True)
    head.close()
    assert cmin >= LAT_COS, cmin
    assert err <= 0.01 * ref.abs().max().item(), err


def test_64_request_batch_requests_match_fp32_oracle(full_head):
    from nanovllm_dots_amd import HipMeanflow
    head, Wb = full_head
    cfg = FULL
    lens, hist, noise = R.synthetic_requests(64, 64, 1024, cfg, seed=0, regime="bf16")
    inp, _, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    n, T = inp.shape[:2]
    M = sum(L + cfg.patch for L in lens)
    print(f"64-request batch: n={n} T={T} M={M} max ctx {max(lens)}", flush=True)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    got = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(g),
             noise=_cuda_bf16(noise)).float().cpu()
    assert torch.isfinite(got).all()
    order = sorted(range(n), key=lambda i: lens[i])
    pick = [order[-1], order[-2], order[0], 0]
    assert lens[order[-1]] >= 1000
    for i in pick:
        ref = R.meanflow_solve_varlen(Wb, cfg, [hist[i]], None, noise[i:i + 1], 4, "fp32")
        _assert_latents(got[i:i + 1], ref, cfg.latent_dim, f"64-request batch: request {i} (c={lens[i]}) vs fp32")


CACHE_ROWS = 600 * 16 + 512


def _cache_inputs(cfg, n=4):
    """bench.py's cached-solve inputs: RandomState(5) rows and noise."""
    rs = np.random.RandomState(5)
    hist = torch.from_numpy(rs.standard_normal((n, CACHE_ROWS, cfg.hidden)).astype(np.float32))
    noise = torch.from_numpy(rs.standard_normal((n, cfg.patch, cfg.latent_dim)).astype(np.float32))
    return R.round_bf16(hist), R.round_bf16(noise)


def _cached_solve(head, hist, noise):
    from nanovllm_dots_amd import HipFMCache
    n, rows, _ = hist.shape
    L = rows - 1
    cache = HipFMCache(head, n, rows + head.spec.patch + 8, 4)
    cache.extend(_cuda_bf16(hist[:, :L]), [L] * n)
    assert cache.lengths == [L] * n
    out = cache.solve(_cuda_bf16(hist[:, L]), noise=_cuda_bf16(noise)).float().cpu()
    cache.close()
    torch.cuda.synchronize()
    return out


def test_cached_solve_10111_rows_vs_fp32_full_recompute(full_head):
    head, Wb = full_head
    cfg = FULL
    hist, noise = _cache_inputs(cfg)
    print(f"cache: one stream, {CACHE_ROWS - 1} cached rows + 1 hidden + {cfg.patch} latent rows", flush=True)
    got = _cached_solve(head, hist[:1], noise[:1])
    ref = _fp32_solve(Wb, cfg, [hist[0]], None, noise[:1], device="cuda")
    torch.cuda.empty_cache()
    _assert_latents(got, ref, cfg.latent_dim, "stream 0 cached vs fp32 full recompute")


def test_four_stream_cache_equals_per_stream_caches(full_head):
    head, _ = full_head
    cfg = FULL
    hist, noise = _cache_inputs(cfg)
    print(f"cache: 4 streams x {CACHE_ROWS - 1} cached rows, batched vs alone", flush=True)
    both = _cached_solve(head, hist, noise)
    for i in range(4):
        solo = _cached_solve(head, hist[i:i + 1], noise[i:i + 1])
        print(f"  stream {i}: bit-identical={torch.equal(solo[0], both[i])}", flush=True)
        _assert_latents(both[i:i + 1], solo, cfg.latent_dim, f"stream {i} batched vs alone")


@pytest.mark.parametrize("K,N", [(1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024)])
@pytest.mark.parametrize("M", [8192, 16384])
def test_w8a8_int32_accumulators_match_int_mm(M, K, N):
    from nanovllm_dots_amd.int8 import gemm_w8a8
    g = torch.Generator(device="cpu").manual_seed(M + 3 * K + N)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).cuda()
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    print(f"w8a8 int32 M={M} K={K} N={N}", flush=True)
    acc = gemm_w8a8(xq, wq, out_int32=True)
    ref = torch._int_mm(xq, wq.t().contiguous())
    assert torch.equal(acc, ref)
