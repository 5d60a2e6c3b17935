"""Prefix K/V cache semantics for a MeanFlow solve (test infrastructure only).

Restates nanovllm_dots/models/dots/cached_fm.py (FMCache :82-114,
extend_cache :118-164, active_forward :167-197) — written there for the CFG
flow-matching DiT — for the MeanFlow DiT, whose condition per solver step is
c_k = T(t_k) + D(dt_k) + g (D/batched_fm.py:113-121) instead of T(t_k) + g.
History rows attend causally among themselves, so at a fixed step their
per-layer K/V do not depend on the latent and are cached per (step, layer);
the 1 + P active rows attend to [cache | themselves] with no mask.
"""
from __future__ import annotations

import torch

from . import dit_ref as R


def _project_qkv(W, cfg, l, x, pos, Rg):
    """q/k/v projection, head split, qk_norm, RoPE (cached_fm.py:44-54)."""
    p = f"blocks.{l}.attn."
    n, H = x.shape
    nh, hd = cfg.heads, cfg.head_dim
    q = Rg.linear(x, W[p + "q_proj.weight"], W.get(p + "q_proj.bias")).view(n, nh, hd)
    k = Rg.linear(x, W[p + "k_proj.weight"], W.get(p + "k_proj.bias")).view(n, nh, hd)
    v = Rg.linear(x, W[p + "v_proj.weight"], W.get(p + "v_proj.bias")).view(n, nh, hd)
    if cfg.qk_norm != "none":
        q = R.qk_norm(q, W, p + "q_norm", cfg)
        k = R.qk_norm(k, W, p + "k_norm", cfg)
    if cfg.rotary:
        cos, sin = R.rope_tables(pos.float(), hd, cfg.rotary_theta)
        q = R.apply_rope(q, cos[:, None], sin[:, None])
        k = R.apply_rope(k, cos[:, None], sin[:, None])
    return Rg.r(q), Rg.r(k), Rg.r(v)


def _attend(q, k, v, allowed, hd, Rg):
    s = torch.einsum("qhd,khd->hqk", q.float(), k.float()) * (hd ** -0.5)
    s = s.masked_fill(~allowed[None], float("-inf"))
    return Rg.r(torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), v.float()))


def _block(W, cfg, l, h, c, pos, kv, causal_from, Rg):
    """One DiTBlock over rows h attending to [cached K/V | own K/V]; own rows are
    causal among themselves when causal_from is not None (extend) and fully
    visible otherwise (active). Returns (h_out, k_full, v_full)."""
    p = f"blocks.{l}."
    H = cfg.hidden
    mod = Rg.linear(R.silu(c, Rg), W[p + "adaLN_modulation.1.weight"], W[p + "adaLN_modulation.1.bias"])
    sh_a, sc_a, g_a, sh_f, sc_f, g_f = [m[None] for m in mod.split(H)]
    q, k, v = _project_qkv(W, cfg, l, R.modulate(R.layer_norm(h, cfg.ln_eps), sh_a, sc_a, Rg), pos, Rg)
    if kv is not None:
        k_full, v_full = torch.cat([kv[0], k]), torch.cat([kv[1], v])
    else:
        k_full, v_full = k, v
    P0, m = k_full.shape[0] - k.shape[0], k.shape[0]
    allowed = torch.ones(m, P0 + m, dtype=torch.bool)
    if causal_from is not None:
        allowed[:, P0:] = torch.ones(m, m, dtype=torch.bool).tril()
    o = _attend(q, k_full, v_full, allowed, cfg.head_dim, Rg).reshape(m, H)
    a = Rg.linear(o, W[p + "attn.o_proj.weight"], W[p + "attn.o_proj.bias"])
    h = Rg.r(h + Rg.r(g_a * a))
    f = Rg.linear(R.modulate(R.layer_norm(h, cfg.ln_eps), sh_f, sc_f, Rg), W[p + "ffn.fc1.weight"],
                  W[p + "ffn.fc1.bias"])
    f = Rg.linear(R.gelu_tanh(f, Rg), W[p + "ffn.fc2.weight"], W[p + "ffn.fc2.bias"])
    return Rg.r(h + Rg.r(g_f * f)), k_full, v_full


class FMCacheRef:
    """cache[k][l] = (K, V) of the prefix rows at step k, layer l (FMCache)."""

    def __init__(self, W, cfg, num_steps: int, g_cond, regime: str = "bf16"):
        self.W, self.cfg, self.S, self.regime = W, cfg, num_steps, regime
        self.Rg = R._R(regime)
        ts, dts = R.meanflow_grid(num_steps, regime)
        self.dts = dts
        g = g_cond[None] if g_cond is not None else None
        self.c = [R.condition(W, cfg, torch.tensor([ts[k]]), torch.tensor([dts[k]]), g, self.Rg)
                  for k in range(num_steps)]
        self.kv = [[None] * cfg.n_blocks for _ in range(num_steps)]
        self.length = 0

    def extend(self, rows):
        """extend_cache (cached_fm.py:118-164) at every step: new prefix rows run
        causally against the cache and persist."""
        W, cfg, Rg = self.W, self.cfg, self.Rg
        m = rows.shape[0]
        pos = torch.arange(self.length, self.length + m, dtype=torch.float32)
        for k in range(self.S):
            h = Rg.linear(rows.float(), W["input_layer.weight"], W["input_layer.bias"])
            for l in range(cfg.n_blocks):
                h, kf, vf = _block(W, cfg, l, h, self.c[k][0], pos, self.kv[k][l], 0, Rg)
                self.kv[k][l] = (kf, vf)
        self.length += m

    def solve(self, last_hidden, noise):
        """MeanFlow steps over the active rows [last hidden | coordinate_proj(z)]
        (active_forward, cached_fm.py:167-197; z update D/batched_fm.py:117-125)."""
        W, cfg, Rg = self.W, self.cfg, self.Rg
        P = cfg.patch
        z = noise.float()
        pos = torch.arange(self.length, self.length + 1 + P, dtype=torch.float32)
        for k in range(self.S):
            zp = Rg.linear(z, W["coordinate_proj.weight"], W["coordinate_proj.bias"])
            x = torch.cat([last_hidden.float()[None], zp])
            h = Rg.linear(x, W["input_layer.weight"], W["input_layer.bias"])
            for l in range(cfg.n_blocks):
                h, _, _ = _block(W, cfg, l, h, self.c[k][0], pos, self.kv[k][l], None, Rg)
            v = R.final_layer(W, cfg, h[1:], self.c[k], Rg)
            z = Rg.r(z + Rg.r(v * self.dts[k]))
        return z
