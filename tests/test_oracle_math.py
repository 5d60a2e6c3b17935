"""Closed forms, brute force and invariants that pin the oracle where the
golden fixtures leave it open (bf16 regime, varlen attention, int8 activation
rounding). CPU only."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import cos_stats
from oracle import dit_ref as R
from oracle import int8_ref as Q


def test_timestep_embedding_closed_form():
    e = R.timestep_embedding(torch.tensor([0.0, 1.0]), 256)
    assert torch.equal(e[0, :128], torch.ones(128)) and torch.equal(e[0, 128:], torch.zeros(128))
    k = torch.arange(128, dtype=torch.float64)
    f = torch.exp(-math.log(10000.0) * k / 128)
    assert torch.allclose(e[1].double(), torch.cat([f.cos(), f.sin()]), atol=1e-6)
    assert R.timestep_embedding(torch.tensor([0.3]), 7).shape == (1, 7)


def test_rope_is_relative_and_matches_complex_rotation():
    """<rope(q, a), rope(k, b)> depends only on a-b; each (d, d+hd/2) pair is the
    complex rotation by pos*inv_freq[d] (rotate_half = cat(-x2, x1))."""
    torch.manual_seed(0)
    hd = 64
    q, k = torch.randn(hd, dtype=torch.float64), torch.randn(hd, dtype=torch.float64)

    def rot(x, p):
        cos, sin = R.rope_tables(torch.tensor([float(p)]), hd, 50000.0)
        return R.apply_rope(x.float()[None], cos, sin)[0].double()

    d1 = rot(q, 10) @ rot(k, 3)
    d2 = rot(q, 107) @ rot(k, 100)
    assert abs(d1 - d2) < 1e-4
    inv = 1.0 / (50000.0 ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    zq = torch.complex(q[:32], q[32:]) * torch.exp(1j * 5.0 * inv)
    r = rot(q, 5)
    assert torch.allclose(r[:32], zq.real, atol=1e-5) and torch.allclose(r[32:], zq.imag, atol=1e-5)


@pytest.mark.parametrize("c", [1, 2, 3, 17])
def test_key_limit_equals_mask_without_padding(c):
    P = 4
    m = R.build_fm_attn_mask(c, c + P, P)
    for r in range(c + P):
        lim = R.fm_key_limit(r, c, P)
        assert m[r, :lim].all() and not m[r, lim:].any()


def test_varlen_attention_brute_force_fp64():
    """Varlen attention (no projection noise: identity q/k/v/o weights) equals a
    per-row fp64 softmax over the allowed key prefix."""
    torch.manual_seed(1)
    cfg = R.DitConfig(hidden=8, heads=2, ffn=16, n_blocks=1, latent_dim=4, patch=2, rotary=False)
    W = {f"blocks.0.attn.{n}_proj.weight": torch.eye(8) for n in "qkvo"}
    W["blocks.0.attn.o_proj.bias"] = torch.zeros(8)
    lens = [3, 1]
    x = torch.randn(sum(lens) + 2 * len(lens), 8)
    out = R.attention_varlen(W, cfg, 0, x, lens, R._R("fp32")).double()
    xd = x.double()
    off = 0
    for c in lens:
        T = c + 2
        for r in range(T):
            lim = R.fm_key_limit(r, c, 2)
            for h in range(2):
                qv = xd[off + r, 4 * h:4 * h + 4]
                ks = xd[off:off + lim, 4 * h:4 * h + 4]
                w = torch.softmax(ks @ qv / 2.0, 0)
                want = w @ ks
                assert torch.allclose(out[off + r, 4 * h:4 * h + 4], want, atol=1e-5)
        off += T


def _small(seed=3):
    cfg = R.DitConfig(hidden=128, heads=2, ffn=256, n_blocks=2, latent_dim=16, patch=4)
    W = R.random_dit_weights(cfg, seed)
    return cfg, W


def test_bf16_regime_tracks_fp32():
    """At full size (12 blocks, hidden 1024, MLP 4096) and on the same
    bf16-valued parameters, the bf16 regime's latents after the NFE=4 solve stay
    within the parity bar of the fixture-pinned fp32 regime: per-row cosine
    >= 0.9999, max |diff| <= 0.02 * max |ref|."""
    cfg = R.DitConfig(hidden=1024, heads=16, ffn=4096, n_blocks=12, latent_dim=64, patch=16)
    Wb = R.weights_for_regime(R.random_dit_weights(cfg, 1), "bf16")
    lens, hist, noise = R.synthetic_requests(2, 64, 160, cfg, seed=3)
    z32 = R.meanflow_solve_varlen(Wb, cfg, hist, None, noise, 4, "fp32")
    zb = R.meanflow_solve_varlen(Wb, cfg, hist, None, noise, 4, "bf16")
    cmin, _ = cos_stats(z32, zb, cfg.latent_dim)
    err = (zb - z32).abs().max().item()
    assert cmin >= 0.9999, cmin
    assert err <= 0.02 * z32.abs().max().item(), err
    # bf16 regime values are bf16-representable
    assert torch.equal(zb, R.round_bf16(zb))


def test_padding_transparency_and_varlen_equality_bf16():
    """Ragged padded batch == each request alone == packed varlen solve."""
    cfg, W = _small()
    Wb = R.weights_for_regime(W, "bf16")
    lens, hist, noise = R.synthetic_requests(3, 3, 24, cfg, seed=4)
    inp, mask, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    zb = R.meanflow_solve(Wb, cfg, inp, mask, pos, g, noise, 4, "bf16")
    zv = R.meanflow_solve_varlen(Wb, cfg, hist, g, noise, 4, "bf16")
    assert cos_stats(zb, zv, cfg.latent_dim)[0] > 0.9999
    for i in range(3):
        i1, m1, p1, g1 = R.pack_fm_inputs([hist[i]], cfg.patch, cfg.hidden)
        z1 = R.meanflow_solve(Wb, cfg, i1, m1, p1, g1, noise[i:i + 1], 4, "bf16")
        assert cos_stats(z1[0], zb[i], cfg.latent_dim)[0] > 0.9999


def test_meanflow_grid_nfe4_exact():
    ts, dts = R.meanflow_grid(4, "bf16")
    assert ts == [0.0, 0.25, 0.5, 0.75] and dts == [0.25] * 4


def test_int8_activation_quant_equals_torch_bf16_ops():
    """The restated fp32-op-then-round sequence == torch's own bf16 tensor ops
    (the form D/int8_dit.py:57-58 is written in)."""
    rs = np.random.RandomState(0)
    x = torch.from_numpy(rs.standard_normal((64, 96)).astype(np.float32)).bfloat16()
    x[0] = 0
    x[1] *= 1e-6
    s_t = (x.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=1e-8)
    q_t = torch.round(x / s_t).clamp(-127, 127).to(torch.int8)
    q, s = Q.quantize_act(x.float())
    assert torch.equal(q, q_t)
    assert torch.equal(s, s_t.float().squeeze(1))


def test_int8_activation_rounds_through_bf16():
    """x/s is rounded to bf16 before round-half-even: a value whose fp32
    quotient rounds up but whose bf16 quotient is a tie must round to even."""
    amax = 125.0                                      # s = bf16(125/127) = 0.984375
    xs = R.round_bf16(torch.linspace(60.0, 120.0, 4001))
    s = R.round_bf16(torch.tensor(amax / 127.0))
    fp32_q = torch.round(xs / s)
    bf16_q = torch.round(R.round_bf16(xs / s))
    differ = xs[fp32_q != bf16_q]
    assert differ.numel() > 0
    x = torch.cat([torch.tensor([amax]), differ])[None]
    q, sc = Q.quantize_act(x)
    assert sc.item() == s.item()
    assert torch.equal(q[0, 1:].float(), bf16_q[fp32_q != bf16_q])
