"""CPU restatement of the reference MeanFlow DiT head (test infrastructure only).

Every function cites the reference file:line it restates. Paths are relative to
the reference repository root; ``D/`` = ``nanovllm_dots/models/dots/`` and
``N/`` = ``nanovllm_dots/models/dots/native/``.

Two numeric regimes:

``fp32``   everything in float32 (the CPU reference path, config "single block
           on CPU").
``bf16``   float32 arithmetic with explicit bf16 rounding at exactly the points
           where the reference rounds when it runs under CUDA autocast(bf16)
           with bf16 parameters (D/engine.py:512, N/loader.py:58-63):
             * nn.Linear: bf16 operands, fp32 accumulate, bias added, one
               rounding to bf16;
             * LayerNorm: computed and returned in fp32 (autocast fp32 op);
             * modulate: fp32 LN output * bf16(1+scale) (+shift), fp32, rounded
               to bf16 only when the next Linear casts it;
             * RoPE in fp32 (autocast disabled, N/layers.py:100, N/layers.py:123),
               q/k rounded to bf16 when SDPA casts them;
             * SDPA: bf16 q/k/v, fp32 softmax, output rounded to bf16;
             * SiLU / GELU(tanh): fp32 math on a bf16 input, bf16 result;
             * the residual stream, gate products, c = T + D + g and the solver
               update z += v*dt are bf16 tensors (one rounding per op).
           Weights are bf16 values (the caller rounds them once).

Tensors passed in and out are float32 holding the regime's values. All
functions are device-agnostic torch code. Tests run them on the CPU; the GPU
parity cases too large for the host (tens of thousands of rows) run the fp32
regime with torch's own float32 kernels on the GPU, never a kernel of the
library under test.
"""
from __future__ import annotations

import math
import zlib
from dataclasses import dataclass, asdict

import numpy as np
import torch


# --------------------------------------------------------------------------- #
# configuration and seeded parameters
# --------------------------------------------------------------------------- #
@dataclass
class DitConfig:
    """Shape of the DiT velocity predictor. Mirrors the ``DiT`` block of the
    checkpoint config read by N/config.py:46-47 / N/loader.py:52-67 plus the core
    scalars of N/core.py:50-55 (latent_dim, latent_patch_size)."""
    hidden: int = 1024
    heads: int = 16
    ffn: int = 4096
    n_blocks: int = 12
    latent_dim: int = 64
    patch: int = 16
    qkv_bias: bool = False
    qk_norm: str = "none"          # "none" | "LayerNorm" | "RMSNorm"  (N/layers.py:156-158)
    rotary: bool = True             # rotary_bias (N/layers.py:164-165)
    rotary_theta: float = 50000.0   # N/layers.py:108, N/layers.py:144
    freq_dim: int = 256             # TimestepEmbedder frequency size (N/dit.py:24)
    meanflow: bool = True           # duration_embedder present (N/dit.py:124-125)
    ln_eps: float = 1e-5            # N/dit.py:68-71, N/dit.py:57

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    def to_dict(self) -> dict:
        return asdict(self)


def param_shapes(cfg: DitConfig) -> dict[str, tuple[int, ...]]:
    """State-dict names and shapes of the reference DiT (N/dit.py:111-133,
    N/layers.py:78-165) plus ``coordinate_proj`` from the core (N/core.py:66).
    Norms with ``modulation=True`` have no affine (N/dit.py:70-71)."""
    H, F, hd, ld = cfg.hidden, cfg.ffn, cfg.head_dim, cfg.latent_dim
    s: dict[str, tuple[int, ...]] = {
        "input_layer.weight": (H, H), "input_layer.bias": (H,),
        "time_embedder.mlp.0.weight": (H, cfg.freq_dim), "time_embedder.mlp.0.bias": (H,),
        "time_embedder.mlp.2.weight": (H, H), "time_embedder.mlp.2.bias": (H,),
    }
    if cfg.meanflow:
        s.update({
            "duration_embedder.mlp.0.weight": (H, cfg.freq_dim),
            "duration_embedder.mlp.0.bias": (H,),
            "duration_embedder.mlp.2.weight": (H, H), "duration_embedder.mlp.2.bias": (H,),
        })
    for l in range(cfg.n_blocks):
        p = f"blocks.{l}."
        for nm in ("q", "k", "v"):
            s[p + f"attn.{nm}_proj.weight"] = (H, H)
            if cfg.qkv_bias:
                s[p + f"attn.{nm}_proj.bias"] = (H,)
        if cfg.qk_norm != "none":
            for nm in ("q", "k"):
                s[p + f"attn.{nm}_norm.weight"] = (hd,)
                if cfg.qk_norm == "LayerNorm":
                    s[p + f"attn.{nm}_norm.bias"] = (hd,)
        s[p + "attn.o_proj.weight"] = (H, H)
        s[p + "attn.o_proj.bias"] = (H,)
        s[p + "ffn.fc1.weight"] = (F, H)
        s[p + "ffn.fc1.bias"] = (F,)
        s[p + "ffn.fc2.weight"] = (H, F)
        s[p + "ffn.fc2.bias"] = (H,)
        s[p + "adaLN_modulation.1.weight"] = (6 * H, H)
        s[p + "adaLN_modulation.1.bias"] = (6 * H,)
    s.update({
        "output_layer.adaLN_modulation.1.weight": (2 * H, H),
        "output_layer.adaLN_modulation.1.bias": (2 * H,),
        "output_layer.linear.weight": (ld, H), "output_layer.linear.bias": (ld,),
        "coordinate_proj.weight": (H, ld), "coordinate_proj.bias": (H,),
    })
    return s


def param_seed(seed: int, name: str) -> int:
    """Per-parameter RandomState seed: independent of iteration order, so any
    module ordering regenerates the same tensors."""
    return (seed * 1_000_003 + zlib.crc32(name.encode())) % (2 ** 32)


def init_param(name: str, shape, seed: int, std: float = 0.02) -> np.ndarray:
    """N(0, std) float32 from a legacy ``RandomState`` stream (frozen across
    numpy versions). qk-norm scales are 1 + N(0, std) so a random-init head is
    not zeroed by its own norm."""
    rng = np.random.RandomState(param_seed(seed, name))
    a = rng.normal(0.0, std, size=shape).astype(np.float32)
    if name.endswith("_norm.weight"):
        a += 1.0
    return a


def random_dit_weights(cfg: DitConfig, seed: int = 0) -> dict[str, torch.Tensor]:
    """All parameters, float32, N(0, 0.02) (weights and biases alike)."""
    return {k: torch.from_numpy(init_param(k, shp, seed)) for k, shp in param_shapes(cfg).items()}


def round_bf16(t: torch.Tensor) -> torch.Tensor:
    """float32 -> nearest-even bf16 -> float32."""
    return t.to(torch.bfloat16).to(torch.float32)


def weights_for_regime(W: dict[str, torch.Tensor], regime: str) -> dict[str, torch.Tensor]:
    """bf16 and int8 regimes: the parameters are bf16 tensors (N/loader.py:58-63)."""
    if regime in ("bf16", "int8"):
        return {k: round_bf16(v.float()) for k, v in W.items()}
    return {k: v.float() for k, v in W.items()}


class _R:
    """Rounding points of one regime. "int8" is the bf16 regime with the DiT
    after quantize_dit_ (D/int8_dit.py:71-85): every linear with
    min(in, out) >= 512 is an Int8DynamicLinear (D/int8_dit.py:34-65)."""

    INT8_MIN_FEATURES = 512

    def __init__(self, regime: str):
        if regime not in ("fp32", "bf16", "int8"):
            raise ValueError(regime)
        self.bf16 = regime in ("bf16", "int8")
        self.int8 = regime == "int8"
        self._wq = {}

    def r(self, t):
        return round_bf16(t) if self.bf16 else t

    def linear(self, x, w, b=None):
        """nn.Linear under autocast: bf16 operands, fp32 accumulate, +bias,
        one rounding (cuBLAS/hipBLASLt bias epilogue); in the int8 regime an
        eligible weight goes through the W8A8 linear instead."""
        if self.int8 and min(w.shape) >= self.INT8_MIN_FEATURES:
            return self._int8_linear(x, w, b)
        y = torch.matmul(self.r(x), w.t())
        if b is not None:
            y = y + b
        return self.r(y)

    def _int8_linear(self, x, w, b):
        """Int8DynamicLinear.forward: per-token bf16 activation quantisation,
        the weight quantised once in float32, the int32 product (exact in
        float64: |acc| < 2^53) converted to float32 as acc.float() does, then
        ((acc * s_x) * s_w) + b rounded to bf16 (oracle/int8_ref.py)."""
        from .int8_ref import dequant, quantize_act, quantize_weight
        key = (w.data_ptr(), tuple(w.shape))
        if key not in self._wq:
            self._wq[key] = quantize_weight(w)
        Wq, s_w = self._wq[key]
        shape = x.shape
        x2 = self.r(x).reshape(-1, shape[-1])
        q, s_x = quantize_act(x2)
        acc = (q.double() @ Wq.double().t()).float()
        y = dequant(acc, s_x, s_w, b)
        return y.reshape(*shape[:-1], w.shape[0])


# --------------------------------------------------------------------------- #
# elementwise pieces
# --------------------------------------------------------------------------- #
def timestep_embedding(t: torch.Tensor, dim: int = 256, max_period: float = 10000.0):
    """N/dit.py:34-43: freqs = exp(-ln(max_period) * k / half), args = t*freqs,
    embedding = [cos(args), sin(args)] (cos first), all float32."""
    half = dim // 2
    freqs = torch.exp(
        -math.log(max_period) * torch.arange(0, half, dtype=torch.float32) / half
    ).to(t.device)
    args = t[:, None].float() * freqs[None]
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    if dim % 2:
        emb = torch.cat([emb, torch.zeros_like(emb[:, :1])], dim=-1)
    return emb


def silu(x, R: _R):
    return R.r(torch.nn.functional.silu(x))


def gelu_tanh(x, R: _R):
    """nn.GELU(approximate="tanh") (N/dit.py:130)."""
    return R.r(torch.nn.functional.gelu(x, approximate="tanh"))


def layer_norm(x, eps: float):
    """LayerNorm without affine (N/dit.py:70-71, N/dit.py:57); fp32 result."""
    return torch.nn.functional.layer_norm(x.float(), (x.shape[-1],), eps=eps)


def modulate(x, shift, scale, R: _R):
    """N/dit.py:19-20 ``x * (1 + scale) + shift`` with per-row shift/scale
    already broadcast to x's shape. ``1 + scale`` is a bf16 op under the bf16
    regime; the product and sum are fp32 because x (a LayerNorm output) is."""
    onep = R.r(1.0 + scale)
    return x * onep + shift


def timestep_mlp(W, prefix: str, t: torch.Tensor, cfg: DitConfig, R: _R):
    """TimestepEmbedder.forward (N/dit.py:45-47): Linear -> SiLU -> Linear."""
    e = timestep_embedding(t, cfg.freq_dim)
    h = R.linear(e, W[prefix + ".mlp.0.weight"], W[prefix + ".mlp.0.bias"])
    h = silu(h, R)
    return R.linear(h, W[prefix + ".mlp.2.weight"], W[prefix + ".mlp.2.bias"])


def condition(W, cfg: DitConfig, timesteps, duration, g_cond, R: _R):
    """c = T(t) [+ D(dt)] [+ g] (N/dit.py:137-143); [B, H]."""
    c = timestep_mlp(W, "time_embedder", timesteps, cfg, R)
    if cfg.meanflow and duration is not None:
        c = R.r(c + timestep_mlp(W, "duration_embedder", duration, cfg, R))
    if g_cond is not None:
        c = R.r(c + g_cond)
    return c


def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """RotaryEmbedding.inv_freq (N/layers.py:110-113), float32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))


def rope_tables(pos: torch.Tensor, head_dim: int, theta: float):
    """RotaryEmbedding.forward (N/layers.py:124-134): freqs = pos (x) inv_freq in
    fp32, emb = cat(freqs, freqs); returns cos, sin of shape pos.shape + [hd]."""
    inv = rope_inv_freq(head_dim, theta).to(pos.device)
    f = pos.float()[..., None] * inv
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(t, cos, sin):
    """apply_rotary_pos_emb / rotate_half (N/layers.py:95-104):
    t*cos + cat(-t2, t1)*sin, in fp32."""
    half = t.shape[-1] // 2
    t1, t2 = t[..., :half], t[..., half:]
    rot = torch.cat([-t2, t1], dim=-1)
    return t.float() * cos + rot.float() * sin


def qk_norm(x, W, name: str, cfg: DitConfig):
    """Per-head q_norm/k_norm (N/layers.py:156-158, :185): LayerNorm(head_dim)
    with affine (eps 1e-5) or RMSNorm(head_dim) (eps = finfo(float32).eps),
    evaluated in fp32."""
    if cfg.qk_norm == "LayerNorm":
        return torch.nn.functional.layer_norm(
            x.float(), (x.shape[-1],), W[name + ".weight"], W[name + ".bias"], eps=1e-5)
    if cfg.qk_norm == "RMSNorm":
        xf = x.float()
        eps = torch.finfo(torch.float32).eps
        return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * W[name + ".weight"]
    return x


# --------------------------------------------------------------------------- #
# padded dense-mask DiT (the reference layout)
# --------------------------------------------------------------------------- #
def attention_padded(W, cfg: DitConfig, l: int, x, mask, pos_ids, R: _R):
    """MultiHeadAttention.forward (N/layers.py:167-208) on [B, T, H] with a
    [B, T, T] bool mask: q/k/v projections, head split, qk_norm, RoPE (fp32),
    additive -inf bias, softmax(q k^T / sqrt(hd)) v, o_proj (with bias)."""
    p = f"blocks.{l}.attn."
    B, T, H = x.shape
    nh, hd = cfg.heads, cfg.head_dim
    q = R.linear(x, W[p + "q_proj.weight"], W.get(p + "q_proj.bias"))
    k = R.linear(x, W[p + "k_proj.weight"], W.get(p + "k_proj.bias"))
    v = R.linear(x, W[p + "v_proj.weight"], W.get(p + "v_proj.bias"))
    q = q.view(B, T, nh, hd).transpose(1, 2)
    k = k.view(B, T, nh, hd).transpose(1, 2)
    v = v.view(B, T, nh, hd).transpose(1, 2)
    if cfg.qk_norm != "none":
        q = qk_norm(q, W, p + "q_norm", cfg)
        k = qk_norm(k, W, p + "k_norm", cfg)
    if cfg.rotary:
        cos, sin = rope_tables(pos_ids, hd, cfg.rotary_theta)   # [B, T, hd]
        q = apply_rope(q, cos[:, None], sin[:, None])
        k = apply_rope(k, cos[:, None], sin[:, None])
    q, k, v = R.r(q), R.r(k), R.r(v)
    s = torch.matmul(q, k.transpose(-1, -2)) * (hd ** -0.5)
    if mask is not None:
        s = s.masked_fill(~mask[:, None], float("-inf"))
    a = torch.softmax(s, dim=-1)
    o = R.r(torch.matmul(a, v))
    o = o.transpose(1, 2).reshape(B, T, H)
    return R.linear(o, W[p + "o_proj.weight"], W[p + "o_proj.bias"])


def block_forward_padded(W, cfg: DitConfig, l: int, x, c, mask, pos_ids, R: _R):
    """DiTBlock.forward with modulation (N/dit.py:81-108). adaLN chunk order
    shift_a, scale_a, gate_a, shift_f, scale_f, gate_f (N/dit.py:86-87)."""
    p = f"blocks.{l}."
    H = cfg.hidden
    mod = R.linear(silu(c, R), W[p + "adaLN_modulation.1.weight"], W[p + "adaLN_modulation.1.bias"])
    sh_a, sc_a, g_a, sh_f, sc_f, g_f = [m[:, None, :] for m in mod.split(H, dim=1)]
    h = modulate(layer_norm(x, cfg.ln_eps), sh_a, sc_a, R)
    a = attention_padded(W, cfg, l, h, mask, pos_ids, R)
    x = R.r(x + R.r(g_a * a))
    h = modulate(layer_norm(x, cfg.ln_eps), sh_f, sc_f, R)
    f = R.linear(h, W[p + "ffn.fc1.weight"], W[p + "ffn.fc1.bias"])
    f = gelu_tanh(f, R)
    f = R.linear(f, W[p + "ffn.fc2.weight"], W[p + "ffn.fc2.bias"])
    return R.r(x + R.r(g_f * f))


def final_layer(W, cfg: DitConfig, x, c, R: _R):
    """FinalLayer.forward (N/dit.py:60-63); x is [..., H] with c broadcast."""
    H = cfg.hidden
    mod = R.linear(silu(c, R), W["output_layer.adaLN_modulation.1.weight"],
                   W["output_layer.adaLN_modulation.1.bias"])
    sh, sc = mod[:, :H], mod[:, H:]
    while sh.dim() < x.dim():
        sh, sc = sh[:, None], sc[:, None]
    h = modulate(layer_norm(x, cfg.ln_eps), sh, sc, R)
    return R.linear(h, W["output_layer.linear.weight"], W["output_layer.linear.bias"])


def dit_forward(W, cfg: DitConfig, x, timesteps, duration, attn_mask, pos_ids, g_cond,
                regime: str = "fp32", return_hidden: bool = False):
    """DiT.forward (N/dit.py:135-148) on the padded layout; returns [B, T, ld]
    (and the last block's hidden state when ``return_hidden``)."""
    R = _R(regime)
    c = condition(W, cfg, timesteps, duration, g_cond, R)
    h = R.linear(x, W["input_layer.weight"], W["input_layer.bias"])
    for l in range(cfg.n_blocks):
        h = block_forward_padded(W, cfg, l, h, c, attn_mask, pos_ids, R)
    out = final_layer(W, cfg, h, c, R)
    return (out, h) if return_hidden else out


# --------------------------------------------------------------------------- #
# FM mask / positions / packing (the input contract of the boundary)
# --------------------------------------------------------------------------- #
def build_fm_attn_mask(fm_seq_len: int, total_len: int, patch: int,
                       hidden_patch_size: int = 1) -> torch.Tensor:
    """DotsModel._build_fm_attn_mask (N/model.py:57-75) for one request, [T, T]
    bool. Rows [0, c-hp) causal among themselves; rows [c-hp, c) and the latent
    rows see [0, c) and the latent slot; padding rows see only themselves."""
    if fm_seq_len <= 0:
        raise RuntimeError("FM sequence length must be positive before decode.")
    m = torch.zeros(total_len, total_len, dtype=torch.bool)
    latent_start = total_len - patch
    bs = fm_seq_len - hidden_patch_size
    if bs > 0:
        m[:bs, :bs] = torch.ones(bs, bs, dtype=torch.bool).tril()
    m[bs:fm_seq_len, :fm_seq_len] = True
    m[bs:fm_seq_len, latent_start:] = True
    m[latent_start:, :fm_seq_len] = True
    m[latent_start:, latent_start:] = True
    if latent_start > fm_seq_len:
        idx = torch.arange(fm_seq_len, latent_start)
        m[idx, idx] = True
    return m


def build_fm_pos_ids(fm_seq_len: int, total_len: int, patch: int) -> torch.Tensor:
    """DotsModel._build_fm_pos_ids (N/model.py:77-87), float32 [T]: history
    0..c-1, latent rows c..c+P-1, padding 0."""
    pos = torch.zeros(total_len, dtype=torch.float32)
    pos[:fm_seq_len] = torch.arange(fm_seq_len, dtype=torch.float32)
    pos[total_len - patch:] = torch.arange(fm_seq_len, fm_seq_len + patch, dtype=torch.float32)
    return pos


def pack_fm_inputs(histories: list[torch.Tensor], patch: int, hidden: int, g_cond=None):
    """DotsBatchEngine._pack_fm_inputs (D/engine.py:635-688), MeanFlow branch,
    no bucketing: histories[i] is [c_i, H]; returns padded ``inp`` [N,T,H]
    (latent slot zero), ``mask`` [N,T,T], ``pos`` [N,T], ``g`` [N,H]."""
    n = len(histories)
    max_len = max(h.shape[0] for h in histories)
    T = max_len + patch
    inp = torch.zeros(n, T, hidden)
    mask = torch.zeros(n, T, T, dtype=torch.bool)
    pos = torch.zeros(n, T)
    for i, h in enumerate(histories):
        L = h.shape[0]
        inp[i, :L] = h
        mask[i] = build_fm_attn_mask(L, T, patch)
        pos[i] = build_fm_pos_ids(L, T, patch)
    g = torch.zeros(n, hidden) if g_cond is None else g_cond.clone()
    return inp, mask, pos, g


def meanflow_grid(num_steps: int, regime: str = "bf16"):
    """``torch.linspace(0, 1, nfe+1)`` in the solver dtype and the per-step
    (t, dt = t[s+1]-t[s]) pairs (D/batched_fm.py:113-116)."""
    dt_ = torch.bfloat16 if regime in ("bf16", "int8") else torch.float32
    times = torch.linspace(0.0, 1.0, num_steps + 1, dtype=dt_)
    ts = [times[s].float().item() for s in range(num_steps)]
    dts = [(times[s + 1] - times[s]).float().item() for s in range(num_steps)]
    return ts, dts


def meanflow_solve(W, cfg: DitConfig, input_sequence, attn_mask, pos_ids, g_cond, noise,
                   num_steps: int = 4, regime: str = "fp32"):
    """batched_meanflow (D/batched_fm.py:82-126): z = noise; per step
    zp = coordinate_proj(z); z_c = input_sequence with the latent slot = zp;
    v = DiT(z_c, t, duration=dt)[:, -P:]; z = z + v*dt. Returns [N, P, ld]."""
    R = _R(regime)
    n, T, _ = input_sequence.shape
    P = cfg.patch
    ts, dts = meanflow_grid(num_steps, regime)
    z = noise.float()
    for s in range(num_steps):
        t = torch.full((n,), ts[s])
        dt = torch.full((n,), dts[s])
        zp = R.linear(z, W["coordinate_proj.weight"], W["coordinate_proj.bias"])
        z_c = input_sequence.float().clone()
        z_c[:, T - P:] = zp
        v = dit_forward(W, cfg, z_c, t, dt, attn_mask, pos_ids, g_cond, regime)[:, T - P:]
        z = R.r(z + R.r(v * dts[s]))
    return z


# --------------------------------------------------------------------------- #
# varlen twin (packed rows, implicit FM mask)
# --------------------------------------------------------------------------- #
def fm_key_limit(r: int, c: int, patch: int, hidden_patch_size: int = 1) -> int:
    """Number of visible keys (a prefix [0, limit)) for packed row r of a
    request with c history rows and ``patch`` latent rows laid out contiguously
    (no padding gap): the implicit form of N/model.py:57-75."""
    bs = c - hidden_patch_size
    return r + 1 if r < bs else c + patch


def attention_varlen(W, cfg: DitConfig, l: int, x, lens: list[int], R: _R):
    """MultiHeadAttention.forward on packed rows; request i occupies
    rows [cu_i, cu_i + c_i + P) with positions 0..c_i+P-1. Runs on x's device;
    the score and value products are float32 matmuls of contiguous operands."""
    p = f"blocks.{l}.attn."
    M, H = x.shape
    dev = x.device
    nh, hd, P = cfg.heads, cfg.head_dim, cfg.patch
    q = R.linear(x, W[p + "q_proj.weight"], W.get(p + "q_proj.bias")).view(M, nh, hd)
    k = R.linear(x, W[p + "k_proj.weight"], W.get(p + "k_proj.bias")).view(M, nh, hd)
    v = R.linear(x, W[p + "v_proj.weight"], W.get(p + "v_proj.bias")).view(M, nh, hd)
    if cfg.qk_norm != "none":
        q = qk_norm(q, W, p + "q_norm", cfg)
        k = qk_norm(k, W, p + "k_norm", cfg)
    out = torch.empty(M, nh, hd, device=dev)
    off = 0
    for c in lens:
        Ti = c + P
        qi, ki, vi = q[off:off + Ti], k[off:off + Ti], v[off:off + Ti]
        if cfg.rotary:
            cos, sin = rope_tables(torch.arange(Ti, dtype=torch.float32, device=dev), hd, cfg.rotary_theta)
            qi = apply_rope(qi, cos[:, None], sin[:, None])
            ki = apply_rope(ki, cos[:, None], sin[:, None])
        qi, ki, vi = R.r(qi), R.r(ki), R.r(vi)
        qh = qi.float().permute(1, 0, 2).contiguous()          # [h, q, d]
        kt = ki.float().permute(1, 2, 0).contiguous()          # [h, d, k]
        s = torch.matmul(qh, kt) * (hd ** -0.5)
        r = torch.arange(Ti, device=dev)
        lim = torch.where(r < c - 1, r + 1, torch.full_like(r, c + P))   # fm_key_limit per row
        allowed = r[None, :] < lim[:, None]
        s = s.masked_fill(~allowed[None], float("-inf"))
        a = torch.softmax(s, dim=-1)
        o = torch.matmul(a, vi.float().permute(1, 0, 2).contiguous())   # [h, q, d]
        out[off:off + Ti] = R.r(o.permute(1, 0, 2))
        off += Ti
    return R.linear(out.reshape(M, H), W[p + "o_proj.weight"], W[p + "o_proj.bias"])


def dit_forward_varlen(W, cfg: DitConfig, x, lens: list[int], timesteps, duration, g_cond,
                       regime: str = "fp32"):
    """DiT.forward on packed rows [M, H] (M = sum(c_i + P)); per-request
    modulation gathered by row. Returns the velocity of every row [M, ld]."""
    R = _R(regime)
    H, P = cfg.hidden, cfg.patch
    c = condition(W, cfg, timesteps, duration, g_cond, R)            # [N, H]
    row_req = torch.cat([torch.full((ci + P,), i, dtype=torch.long) for i, ci in enumerate(lens)]).to(x.device)
    h = R.linear(x, W["input_layer.weight"], W["input_layer.bias"])
    for l in range(cfg.n_blocks):
        p = f"blocks.{l}."
        mod = R.linear(silu(c, R), W[p + "adaLN_modulation.1.weight"],
                       W[p + "adaLN_modulation.1.bias"])[row_req]
        sh_a, sc_a, g_a, sh_f, sc_f, g_f = mod.split(H, dim=1)
        a = attention_varlen(W, cfg, l, modulate(layer_norm(h, cfg.ln_eps), sh_a, sc_a, R), lens, R)
        h = R.r(h + R.r(g_a * a))
        f = R.linear(modulate(layer_norm(h, cfg.ln_eps), sh_f, sc_f, R),
                     W[p + "ffn.fc1.weight"], W[p + "ffn.fc1.bias"])
        f = R.linear(gelu_tanh(f, R), W[p + "ffn.fc2.weight"], W[p + "ffn.fc2.bias"])
        h = R.r(h + R.r(g_f * f))
    return final_layer(W, cfg, h, c[row_req], R)


def meanflow_solve_varlen(W, cfg: DitConfig, histories: list[torch.Tensor], g_cond, noise,
                          num_steps: int = 4, regime: str = "fp32"):
    """The MeanFlow solve on packed rows; equal to ``meanflow_solve`` on the
    padded layout of the same requests (padding transparency). Runs on the
    device of ``noise`` (weights, histories and g_cond must live there too)."""
    R = _R(regime)
    P = cfg.patch
    n = len(histories)
    dev = noise.device
    lens = [h.shape[0] for h in histories]
    ts, dts = meanflow_grid(num_steps, regime)
    z = noise.float()
    patch_rows = []
    off = 0
    for ci in lens:
        patch_rows.append(torch.arange(off + ci, off + ci + P))
        off += ci + P
    patch_rows = torch.cat(patch_rows).to(dev)
    base = torch.cat([torch.cat([h.float(), torch.zeros(P, h.shape[1], device=dev)]) for h in histories])
    for s in range(num_steps):
        zp = R.linear(z, W["coordinate_proj.weight"], W["coordinate_proj.bias"])
        xs = base.clone()
        xs[patch_rows] = zp.reshape(n * P, -1)
        v = dit_forward_varlen(W, cfg, xs, lens, torch.full((n,), ts[s], device=dev),
                               torch.full((n,), dts[s], device=dev), g_cond, regime)
        v = v[patch_rows].reshape(n, P, -1)
        z = R.r(z + R.r(v * dts[s]))
    return z


# --------------------------------------------------------------------------- #
# synthetic workloads (seeded numpy RandomState streams)
# --------------------------------------------------------------------------- #
def synthetic_requests(n: int, ctx_lo: int, ctx_hi: int, cfg: DitConfig, seed: int,
                       llm_width: int | None = None, W=None, regime: str = "bf16"):
    """Context lengths ~ U{ctx_lo..ctx_hi}, histories N(0,1) (optionally
    ``hidden_proj`` of N(0,1) states of width ``llm_width``: N/core.py:67,
    N/model.py:101-110), noise N(0,1). One RandomState stream per kind."""
    rl = np.random.RandomState(seed * 4 + 1)
    ra = np.random.RandomState(seed * 4 + 2)
    rn = np.random.RandomState(seed * 4 + 3)
    lens = [int(x) for x in rl.randint(ctx_lo, ctx_hi + 1, size=n)]
    hist = []
    R = _R("bf16" if regime == "int8" else regime)   # hidden_proj is not a DiT linear
    if llm_width is not None:
        hw = torch.from_numpy(init_param("hidden_proj.weight", (cfg.hidden, llm_width), seed))
        hb = torch.from_numpy(init_param("hidden_proj.bias", (cfg.hidden,), seed))
        if regime in ("bf16", "int8"):
            hw, hb = round_bf16(hw), round_bf16(hb)
    for L in lens:
        if llm_width is None:
            h = torch.from_numpy(ra.standard_normal((L, cfg.hidden)).astype(np.float32))
            hist.append(R.r(h))
        else:
            s = torch.from_numpy(ra.standard_normal((L, llm_width)).astype(np.float32))
            hist.append(R.linear(s, hw, hb))
    noise = torch.from_numpy(rn.standard_normal((n, cfg.patch, cfg.latent_dim)).astype(np.float32))
    return lens, hist, R.r(noise)


def dit_gemm_flops(cfg: DitConfig, M: int) -> int:
    """Block GEMM FLOPs for M tokens: n_blocks * 2*M*(4H^2 + 2HF)."""
    H, F = cfg.hidden, cfg.ffn
    return cfg.n_blocks * 2 * M * (4 * H * H + 2 * H * F)
