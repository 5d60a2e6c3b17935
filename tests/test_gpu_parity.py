"""HIP path vs the oracle through the C ABI. GPU only.

Two oracle regimes, both on the same bf16-valued parameters and inputs as the
HIP head (the reference loads its checkpoint as bf16, N/loader.py:58-63):

* fp32 — the reference's CPU path, pinned bit for bit by fixtures the
  reference's own DiT wrote (tests/golden). This is the parity bar: latents
  after the full NFE=4 solve reach per-row cosine >= 0.9999 and
  max |diff| <= 0.02 * max |ref|. One DiT forward's velocities (not latents)
  reach per-row cosine >= 0.9998 and the same max |diff|: on the full-size
  forward the bf16 restatement itself reaches only 0.99992 against fp32.
* bf16 — the fp32 oracle with bf16 rounding where CUDA autocast rounds; the HIP
  path tracks it more closely (same bars). Its rounding points are the
  oracle's own reading of autocast, so no parity claim rests on it alone.

The bf16 GEMM's float32 output must match torch's fp32 matmul of the same bf16
operands to 1e-5 relative (accumulation order is the only difference)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from conftest import cos_stats
from oracle import dit_ref as R

pytestmark = pytest.mark.gpu

LAT_COS = 0.9999
LAT_MAXABS_FRAC = 0.02
FWD_FP32_COS = 0.9998   # one forward's velocities against the fp32 oracle


def _head(cfg, seed=0):
    from nanovllm_dots_amd import FMSpec, HipFMHead
    W = R.random_dit_weights(cfg, seed)
    head = HipFMHead(FMSpec.of(cfg), W, device="cuda")
    return head, R.weights_for_regime(W, "bf16")


def _inputs(cfg, n, lo, hi, seed):
    lens, hist, noise = R.synthetic_requests(n, lo, hi, cfg, seed)
    inp, mask, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    return lens, hist, noise, inp, mask, pos, g


def _cuda_bf16(t):
    return t.to(device="cuda", dtype=torch.bfloat16).contiguous()


def _assert_latents(got, ref, ld, label, cos_bar=LAT_COS):
    got, ref = got.float().cpu(), ref.float().cpu()
    cmin, cmean = cos_stats(got, ref, ld)
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    print(f"{label}: cos min {cmin:.6f} mean {cmean:.6f} maxabs {err:.4g} (|ref| {scale:.3g})", flush=True)
    assert cmin >= cos_bar, f"{label}: cos min {cmin:.6f}"
    assert err <= LAT_MAXABS_FRAC * scale, f"{label}: max abs {err}"


def _fp32_solve(Wb, cfg, hist, g, noise, device="cpu"):
    """The fp32 oracle's MeanFlow solve of the requests ``hist`` (packed rows,
    padding-transparent, so equal to the padded solve) on ``device``."""
    dev = torch.device(device)
    Wd = {k: v.to(dev) for k, v in Wb.items()} if dev.type != "cpu" else Wb
    hd = [h.float().to(dev) for h in hist]
    gd = g.float().to(dev) if g is not None else None
    assert not torch.backends.cuda.matmul.allow_tf32   # full float32 products
    with torch.no_grad():
        return R.meanflow_solve_varlen(Wd, cfg, hd, gd, noise.float().to(dev), 4, "fp32").cpu()


def _assert_vs_fp32(got, Wb, cfg, hist, g, noise, label, device="cpu"):
    """HIP latents vs the fixture-pinned fp32 oracle at the parity bar."""
    _assert_latents(got, _fp32_solve(Wb, cfg, hist, g, noise, device), cfg.latent_dim, label + " vs fp32")


# ----------------------------------------------------------------------------- GEMM
GEMM_CASES = [(1, 64, 64, 3), (37, 128, 256, 2), (300, 1024, 1024, -1), (700, 1024, 1024, 0),
              (1000, 3072, 1024, 1), (513, 1024, 4096, -1), (64, 75776 // 8, 1024, -1),
              (777, 512, 1024, 4), (1500, 4096, 1024, 0), (20, 256, 64, 0), (333, 256, 192, 1),
              (1111, 1024, 1024, 5), (600, 1024, 4096, 6), (259, 512, 1024, 7), (1234, 3072, 1024, 1),
              (100, 512, 96, 7), (70, 256, 160, 5), (1500, 4096, 1024, 8), (3001, 1024, 4096, 8),
              (20, 256, 64, 8),
              # tile 9 (4 waves, AGPR accumulators, BK 32 x 5 stages): K steps 1, 2, 3, 4, 5 exercise the
              # guarded prologue / tail paths, the larger ones the unrolled steady state
              (1500, 4096, 1024, 9), (3001, 1024, 4096, 9), (700, 512, 32, 9), (333, 256, 64, 9),
              (37, 256, 96, 9), (300, 768, 128, 9), (513, 256, 160, 9), (2000, 1024, 2048, 9),
              # tiles 10 / 11 (128-row blocks, 32 / 64 columns): decode-sized batches, and past 128 rows
              (68, 1024, 4096, 10), (1, 1024, 1024, 10), (97, 32, 192, 10), (200, 512, 1024, 10),
              (128, 3072, 1024, 11), (33, 128, 640, 11), (300, 256, 128, 11)]


@pytest.mark.parametrize("M,N,K,tile", GEMM_CASES)
def test_gemm_f32_out_matches_torch(M, N, K, tile):
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N)
    A = torch.randn(M, K, generator=g).bfloat16().cuda()
    B = (0.05 * torch.randn(N, K, generator=g)).bfloat16().cuda()
    bias = (0.1 * torch.randn(N, generator=g)).bfloat16().cuda()
    out = torch.empty(M, N, device="cuda", dtype=torch.float32)
    print(f"gemm M={M} N={N} K={K} tile={tile}", flush=True)
    _lib.check(lib.dfh_gemm_bf16(_lib.ptr(A), K, _lib.ptr(B), K, _lib.ptr(out), N, _lib.ptr(bias),
                                 M, N, K, 4, tile, _lib.stream_ptr()))
    ref = A.float() @ B.float().t() + bias.float()
    torch.cuda.synchronize()
    rel = ((out - ref).abs().max() / ref.abs().max()).item()
    assert rel < 1e-5, rel


@pytest.mark.parametrize("tile", [-1, 9])
@pytest.mark.parametrize("epi", [0, 1])
def test_gemm_bf16_epilogues(epi, tile):
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    M, N, K = 333 if tile < 0 else 3333, 512, 1024
    g = torch.Generator(device="cpu").manual_seed(epi)
    A = torch.randn(M, K, generator=g).bfloat16().cuda()
    B = (0.03 * torch.randn(N, K, generator=g)).bfloat16().cuda()
    bias = (0.1 * torch.randn(N, generator=g)).bfloat16().cuda()
    out = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    _lib.check(lib.dfh_gemm_bf16(_lib.ptr(A), K, _lib.ptr(B), K, _lib.ptr(out), N, _lib.ptr(bias),
                                 M, N, K, epi, tile, _lib.stream_ptr()))
    pre = (A.float() @ B.float().t() + bias.float()).bfloat16().float()
    ref = pre
    if epi == 1:
        ref = torch.nn.functional.gelu(pre, approximate="tanh").bfloat16().float()
    torch.cuda.synchronize()
    diff = (out.float() - ref).abs()
    # the pre-activation may differ by one bf16 ulp (accumulation order); GELU's
    # slope is within [-0.2, 1.2], then one more output rounding
    tol = pre.abs() * 2 ** -7 * (1.2 if epi == 1 else 1.0) + ref.abs() * 2 ** -8 + 1e-6
    assert (diff <= tol).all(), diff.max()


# ----------------------------------------------------------------------------- DiT / solve
SMALL = dict(hidden=256, heads=4, ffn=1024, n_blocks=2, latent_dim=64, patch=16)
VARIANTS = {
    "rope": R.DitConfig(**SMALL),
    "qknorm_bias": R.DitConfig(**SMALL, qkv_bias=True, qk_norm="LayerNorm"),
    "rms_norope": R.DitConfig(**SMALL, qk_norm="RMSNorm", rotary=False),
    # q|k|v bias without qk-norm: the QKV epilogue with counted stores and its bias
    "bias_rope": R.DitConfig(**SMALL, qkv_bias=True),
}


@pytest.mark.parametrize("name", list(VARIANTS))
def test_dit_forward_matches_oracle(name):
    from nanovllm_dots_amd import HipDiT
    cfg = VARIANTS[name]
    head, Wb = _head(cfg, seed=3)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 3, 1, 150, seed=5)
    n, T = inp.shape[0], inp.shape[1]
    rs = np.random.RandomState(9)
    x = inp.clone()
    x[:, T - cfg.patch:] = R.round_bf16(torch.from_numpy(rs.standard_normal((n, cfg.patch, cfg.hidden)).astype(np.float32)))
    t = R.round_bf16(torch.from_numpy(rs.uniform(0, 1, n).astype(np.float32)))
    dur = R.round_bf16(torch.from_numpy(rs.uniform(0, 1, n).astype(np.float32)))
    gc = R.round_bf16(torch.from_numpy(0.5 * rs.standard_normal((n, cfg.hidden)).astype(np.float32)))
    print(f"dit_forward {name} lens={lens}", flush=True)
    ref = R.dit_forward(Wb, cfg, x, t, dur, mask, pos, gc, regime="bf16")
    ref32 = R.dit_forward(Wb, cfg, x, t, dur, mask, pos, gc, regime="fp32")
    got = HipDiT(head=head, strict=True)(x=_cuda_bf16(x), timesteps=t.cuda(), duration=dur.cuda(),
                                         attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(gc))
    got = got.float().cpu()
    for i, L in enumerate(lens):
        rows = list(range(L)) + list(range(T - cfg.patch, T))
        cmin, _ = cos_stats(got[i, rows], ref[i, rows])
        c32, _ = cos_stats(got[i, rows], ref32[i, rows])
        print(f"  request {i} (c={L}): cos min {cmin:.6f} vs bf16, {c32:.6f} vs fp32", flush=True)
        assert cmin >= LAT_COS, (i, L, cmin)
        assert c32 >= FWD_FP32_COS, (i, L, c32)
        pad = [r for r in range(T) if r not in rows]
        assert torch.all(got[i, pad] == 0)


@pytest.mark.parametrize("name", list(VARIANTS))
def test_meanflow_solve_matches_oracle(name):
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS[name]
    head, Wb = _head(cfg, seed=4)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 4, 1, 200, seed=6)
    print(f"meanflow {name} lens={lens}", flush=True)
    ref = R.meanflow_solve(Wb, cfg, inp, mask, pos, g, noise, 4, "bf16")
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    got = mf(input_sequence=_cuda_bf16(inp), attn_mask=mask.cuda(), pos_ids=pos.cuda(),
             g_cond=_cuda_bf16(g), noise=_cuda_bf16(noise))
    _assert_latents(got, ref, cfg.latent_dim, f"meanflow-{name}")
    _assert_vs_fp32(got, Wb, cfg, hist, g, noise, f"meanflow-{name}")


def test_edge_lengths_and_a_long_request_match_fp32_oracle():
    """Histories at the 64-key and 128-query tile edges (1, 63, 64, 65, 127,
    128, 129 rows) and one long request (3,000 rows: 24 query tiles, a work-list
    bucket of its own, 47 key tiles) in one batch, padded and varlen, against
    the fp32 oracle's solve of the same requests."""
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS["rope"]
    head, Wb = _head(cfg, seed=21)
    lens = [1, 63, 64, 65, 127, 128, 129, 3000]
    rng = np.random.RandomState(21)
    hist = [R.round_bf16(torch.from_numpy(rng.standard_normal((L, cfg.hidden)).astype(np.float32))) for L in lens]
    noise = R.round_bf16(torch.from_numpy(
        rng.standard_normal((len(lens), cfg.patch, cfg.latent_dim)).astype(np.float32)))
    inp, _, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    print(f"edge lengths {lens}", flush=True)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    got = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(g),
             noise=_cuda_bf16(noise))
    _assert_vs_fp32(got, Wb, cfg, hist, g, noise, "edge lengths")
    vl = head.solve_varlen([_cuda_bf16(h) for h in hist], lens, _cuda_bf16(g), _cuda_bf16(noise), 4, strict=True)
    assert torch.equal(vl, got)


def test_padding_transparency_bit_exact():
    """A ragged batch gives each request bit-identical latents to a solo run."""
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS["rope"]
    head, _ = _head(cfg, seed=7)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 5, 1, 180, seed=8)
    batched = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(),
                 g_cond=_cuda_bf16(g), noise=_cuda_bf16(noise))
    for i in range(5):
        i1, m1, p1, g1 = R.pack_fm_inputs([hist[i]], cfg.patch, cfg.hidden)
        solo = mf(input_sequence=_cuda_bf16(i1), attn_mask=None, pos_ids=p1.cuda(), g_cond=_cuda_bf16(g1),
                  noise=_cuda_bf16(noise[i:i + 1]))
        assert torch.equal(solo[0], batched[i]), i


def test_shape_changes_without_recapture_and_shrink():
    """Successive calls with different (N, T) — growing and shrinking — each
    match the oracle; nothing is captured."""
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS["rope"]
    head, Wb = _head(cfg, seed=11)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    for k, (n, lo, hi) in enumerate([(2, 3, 30), (6, 50, 260), (1, 1, 1), (3, 10, 90)]):
        lens, hist, noise, inp, mask, pos, g = _inputs(cfg, n, lo, hi, seed=20 + k)
        ref = R.meanflow_solve(Wb, cfg, inp, mask, pos, g, noise, 4, "bf16")
        got = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(),
                 g_cond=_cuda_bf16(g), noise=_cuda_bf16(noise))
        _assert_latents(got, ref, cfg.latent_dim, f"shape{k} n={n}")
        _assert_vs_fp32(got, Wb, cfg, hist, g, noise, f"shape{k} n={n}")


def test_nfe_mismatch_and_bad_layout_raise():
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS["rope"]
    head, _ = _head(cfg, seed=1)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 2, 5, 9, seed=1)
    with pytest.raises(RuntimeError, match="nfe"):
        mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=None,
           num_steps=3, noise=_cuda_bf16(noise))
    bad = pos.clone()
    bad[0, -cfg.patch] = 0.0   # history length 0 is not a valid FM layout
    with pytest.raises(RuntimeError, match="valid FM layout"):
        mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=bad.cuda(), g_cond=None,
           noise=_cuda_bf16(noise))
    # the handle stays usable after a rejected input
    out = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=None,
             noise=_cuda_bf16(noise))
    assert torch.isfinite(out.float()).all()


def test_noise_drawn_from_torch_rng_when_absent():
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS["rope"]
    head, _ = _head(cfg, seed=2)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 2, 5, 40, seed=2)
    torch.manual_seed(123)
    a = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=None)
    torch.manual_seed(123)
    nz = torch.randn((2, cfg.patch, cfg.latent_dim), device="cuda", dtype=torch.bfloat16)
    b = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=None, noise=nz)
    assert torch.equal(a, b)


def test_profile_class_mask_and_sample_stride():
    """Dispatch events per class: with every = 1 each launch of every class
    carries them; with a class mask and every = 3, launches 0, 3, 6, ... of
    that class (counted across calls) and nothing else. The events do not
    change the latents; every < 1 is an error."""
    cfg = VARIANTS["rope"]  # 2 blocks: block 0 full rows, block 1 the latent tail
    head, _ = _head(cfg, seed=5)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 3, 20, 90, seed=5)
    args = (_cuda_bf16(inp), pos.cuda(), _cuda_bf16(g), _cuda_bf16(noise), 4)
    ref = head.solve(*args)
    head.profile(True)
    head.profile_read()
    a = head.solve(*args)
    torch.cuda.synchronize()
    full = head.profile_read()
    n_fc1 = full["fc1_gemm"][1]
    print(f"profile: per-class launches {({k: v[1] for k, v in full.items()})}", flush=True)
    assert n_fc1 == 4  # one full-row block per step
    assert full["latent_tail"][1] > 0 and full["attention"][1] > 0
    assert all(ms > 0 for ms, cnt in full.values() if cnt)
    head.profile(True, classes=("fc1_gemm",), every=3)
    b = head.solve(*args)
    c = head.solve(*args)
    torch.cuda.synchronize()
    part = head.profile_read()
    head.profile(False)
    assert part["fc1_gemm"][1] == (2 * n_fc1 + 2) // 3  # launches 0, 3, 6 of the two solves' 8
    assert all(cnt == 0 for k, (ms, cnt) in part.items() if k != "fc1_gemm")
    assert torch.equal(a, ref) and torch.equal(b, ref) and torch.equal(c, ref)
    with pytest.raises(RuntimeError, match="every"):
        head.profile(True, classes=("fc1_gemm",), every=0)


# ----------------------------------------------------------------------------- full size
FULL = R.DitConfig(hidden=1024, heads=16, ffn=4096, n_blocks=12, latent_dim=64, patch=16)


def test_full_size_one_step_forward_8_requests():
    """8 requests, contexts U{64..512} projected from 1536-d N(0,1) states, one
    DiT forward at t=0, dt=0.25 (12 blocks, H=1024)."""
    from nanovllm_dots_amd import HipDiT
    cfg = FULL
    head, Wb = _head(cfg, seed=0)
    lens, hist, noise = R.synthetic_requests(8, 64, 512, cfg, seed=0, llm_width=1536)
    inp, mask, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    n, T = inp.shape[:2]
    zp = R._R("bf16").linear(noise, Wb["coordinate_proj.weight"], Wb["coordinate_proj.bias"])
    x = inp.clone()
    x[:, T - cfg.patch:] = zp
    t = torch.zeros(n)
    dt = torch.full((n,), 0.25)
    print(f"8-request forward lens={lens}", flush=True)
    ref = R.dit_forward(Wb, cfg, x, t, dt, mask, pos, g, regime="bf16")[:, T - cfg.patch:]
    ref32 = R.dit_forward(Wb, cfg, x, t, dt, mask, pos, g, regime="fp32")[:, T - cfg.patch:]
    got = HipDiT(head=head)(x=_cuda_bf16(x), timesteps=t.cuda(), duration=dt.cuda(), pos_ids=pos.cuda(),
                            g_cond=_cuda_bf16(g))[:, T - cfg.patch:]
    _assert_latents(got, ref, cfg.latent_dim, "8-request forward")
    _assert_latents(got, ref32, cfg.latent_dim, "8-request forward vs fp32", cos_bar=FWD_FP32_COS)


def test_full_size_nfe4_solve():
    """Full 12-block NFE=4 solve, 4 requests with contexts U{64..384}."""
    from nanovllm_dots_amd import HipMeanflow
    cfg = FULL
    head, Wb = _head(cfg, seed=1)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 4, 64, 384, seed=3)
    print(f"full solve lens={lens}", flush=True)
    ref = R.meanflow_solve_varlen(Wb, cfg, hist, g, noise, 4, "bf16")
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    got = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(g),
             noise=_cuda_bf16(noise))
    _assert_latents(got, ref, cfg.latent_dim, "full-nfe4")
    _assert_vs_fp32(got, Wb, cfg, hist, g, noise, "full-nfe4")


@pytest.mark.parametrize("M,K,N,tile,epi", [(36937, 4096, 1024, 8, 4), (36937, 1024, 4096, 8, 1),
                                            # fewer tiles than resident workgroups: every tile is split
                                            (68, 4096, 1024, 3, 4), (68, 1024, 4096, 3, 1), (68, 1024, 1024, 3, 0),
                                            (1024, 1024, 4096, 2, 4), (1024, 4096, 1024, 3, 4), (5, 4096, 256, 3, 4),
                                            # the O projection and QKV shapes at 36,937 rows; a 9000-row O
                                            (36937, 1024, 1024, 2, 4), (36937, 1024, 3072, 8, 0),
                                            (9000, 1024, 1024, 2, 1),
                                            (20000, 1024, 4096, 0, 4), (3000, 2048, 256, 3, 4),
                                            (700, 1024, 256, 3, 0),
                                            # the cached solve's decode-sized GEMMs on the 128-row tiles
                                            (68, 4096, 1024, 10, 4), (68, 1024, 4096, 10, 1), (68, 1024, 1024, 10, 0),
                                            (68, 1024, 3072, 11, 0), (100, 4096, 256, 10, 4), (128, 2048, 512, 11, 4)])
def test_gemm_ksplit_matches_whole_tiles(M, K, N, tile, epi):
    """bf16 GEMM with the K-split workspace vs without (float32 sums in a
    different order: f32 output to 1e-5 relative, bf16 output to one ulp)."""
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    g = torch.Generator(device="cpu").manual_seed(M + N)
    A = torch.randn(M, K, generator=g).bfloat16().cuda()
    B = (0.02 * torch.randn(N, K, generator=g)).bfloat16().cuda()
    bias = (0.1 * torch.randn(N, generator=g)).bfloat16().cuda()
    dt = torch.float32 if epi == 4 else torch.bfloat16
    ws = torch.zeros((1 << 27) + (1 << 16), dtype=torch.uint8, device="cuda")  # zero-filled before first use
    outs = []
    for use_ws in (False, True):
        C = torch.zeros((M, N), device="cuda", dtype=dt)
        print(f"gemm ksplit M={M} K={K} N={N} tile={tile} epi={epi} ws={use_ws}", flush=True)
        _lib.check(lib.dfh_gemm_bf16_ws(_lib.ptr(A), K, _lib.ptr(B), K, _lib.ptr(C), N, _lib.ptr(bias), M, N, K,
                                        epi, tile, _lib.ptr(ws) if use_ws else None, ws.numel() if use_ws else 0,
                                        _lib.stream_ptr()), "dfh_gemm_bf16_ws")
        outs.append(C.float().cpu())
    whole, split = outs
    if epi == 4:
        assert torch.allclose(split, whole, rtol=1e-5, atol=1e-5 * whole.abs().max().item())
    else:
        # one f32 ulp of the sum can flip the bf16 rounding of the (pre-activation) value:
        # a bf16 ulp of the pre-activation (through GELU' <= 1.13) plus one of the output
        pre = (A.float() @ B.float().t() + bias.float()).abs().cpu()
        tol = pre * 2.0 ** -7 * 1.2 + whole.abs() * 2.0 ** -8 + 1e-6
        assert ((split - whole).abs() <= tol).all()
