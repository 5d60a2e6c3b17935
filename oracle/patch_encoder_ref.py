"""CPU restatement of the patch encoder's per-patch decode (test infrastructure:
only tests/, bench.py's CPU leg and smoke() use it, as the checker).

The patch encoder (VAESemanticEncoder) turns each generated latent patch into the
LLM's next input embedding:

  * causal downsample step: conv1d (kernel 2, stride 2) over [conv_tail, patch]
    frames, then in_proj -> out_ds_rate = patch / 2 tokens
    (nanovllm_dots/models/dots/native/patch_encoder.py:229-236, the Conv1d of
    native/layers.py:30-50 with left_padding = 1);
  * SuperviseEncoder.decode_step over the encoder layers
    (native/patch_encoder.py:77-85, 137-142): per layer x += attn(LN(x)),
    x += MLP_SiLU(LN(x)), LayerNorm with affine parameters, eps 1e-5;
  * MultiHeadAttention.decode_step (native/layers.py:210-249): q, k, v
    projections without bias (the encoder layers build MultiHeadAttention with
    its defaults: qkv_bias, qk_norm and rotary_bias all off,
    native/patch_encoder.py:28-37), the block's k / v written at its positions,
    then attention of the block over keys <= its own position (the cache's
    earlier rows and the causal block), o_proj with bias;
  * _project_embeddings (native/patch_encoder.py:222-225): the out_ds_rate
    tokens concatenated, out_proj -> [1, out_dim].

FlashPatchEncoder.decode_patch (nanovllm_dots/models/dots/flash_patch_encoder.py
:103-139) runs the same per-patch computation for n requests at once, request i
in cache row rows[i] with its own history length; PatchEncoderCacheRef restates
that bookkeeping (per-row conv tail, cache and length) over the per-request
decode, which is exactly how the reference's own test compares the two
(tests/test_patch_encoder.py:20-54).

Parity: the float32 decode is pinned by tests/golden/patch_encoder.npz, written
by the reference's own native/patch_encoder.py (tests/golden/gen_golden.py).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .dit_ref import init_param


@dataclass(frozen=True)
class PatchEncConfig:
    """SuperviseEncoder defaults (native/patch_encoder.py:88-97): hidden 1024,
    16 heads, MLP 4096, 6 layers, LayerNorm; latent patch of 16 frames x 64."""
    latent_dim: int = 64
    patch: int = 16
    hidden: int = 1024
    heads: int = 16
    ffn: int = 4096
    n_layers: int = 6
    out_dim: int = 1536
    ln_eps: float = 1e-5

    @property
    def ods(self) -> int:  # out_ds_rate (native/patch_encoder.py:151)
        return self.patch // 2

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def pe_param_shapes(cfg: PatchEncConfig) -> dict[str, tuple]:
    """State-dict names and shapes of VAESemanticEncoder (native/patch_encoder.py:144-152)."""
    H, F_, L = cfg.hidden, cfg.ffn, cfg.latent_dim
    s = {"ds_proj.weight": (L, L, 2), "ds_proj.bias": (L,), "in_proj.weight": (H, L), "in_proj.bias": (H,),
         "out_proj.weight": (cfg.out_dim, H * cfg.ods), "out_proj.bias": (cfg.out_dim,)}
    for l in range(cfg.n_layers):
        p = f"encoder.layers.{l}."
        for n in ("q_proj", "k_proj", "v_proj"):
            s[p + f"attn.{n}.weight"] = (H, H)
        s[p + "attn.o_proj.weight"] = (H, H)
        s[p + "attn.o_proj.bias"] = (H,)
        for n in ("attn_norm", "ffn_norm"):
            s[p + f"{n}.weight"] = (H,)
            s[p + f"{n}.bias"] = (H,)
        s[p + "ffn.fc1.weight"] = (F_, H)
        s[p + "ffn.fc1.bias"] = (F_,)
        s[p + "ffn.fc2.weight"] = (H, F_)
        s[p + "ffn.fc2.bias"] = (H,)
    return s


def random_pe_weights(cfg: PatchEncConfig, seed: int = 0) -> dict[str, torch.Tensor]:
    """N(0, 0.02) float32 for every parameter; the LayerNorm scales are 1 + N(0, 0.02)."""
    return {k: torch.from_numpy(init_param(k, shp, seed)) for k, shp in pe_param_shapes(cfg).items()}


@dataclass
class DecodeState:
    """One request's decode state (native/patch_encoder.py:21-25): conv tail
    [latent_dim, 1], per-layer key / value caches [heads, cap, head_dim], length."""
    conv_tail: torch.Tensor
    k: list
    v: list
    seq_len: int = 0


def init_state(cfg: PatchEncConfig, cap: int) -> DecodeState:
    z = lambda: torch.zeros(cfg.heads, cap, cfg.head_dim)
    return DecodeState(torch.zeros(cfg.latent_dim, 1), [z() for _ in range(cfg.n_layers)],
                       [z() for _ in range(cfg.n_layers)], 0)


def downsample_step(W, cfg: PatchEncConfig, patch: torch.Tensor, tail: torch.Tensor):
    """patch [P, latent_dim] -> (in_proj(conv) [P/2, hidden], new tail [latent_dim, 1])
    (native/patch_encoder.py:229-236)."""
    raw = patch.t()                                   # [latent_dim, P]
    conv_in = torch.cat([tail, raw], dim=-1)[None]    # [1, latent_dim, P + 1]
    y = F.conv1d(conv_in, W["ds_proj.weight"], W["ds_proj.bias"], stride=2)[0].t()   # [P/2, latent_dim]
    return F.linear(y, W["in_proj.weight"], W["in_proj.bias"]), raw[:, -1:].clone()


def layer_decode(W, cfg: PatchEncConfig, l: int, x: torch.Tensor, st: DecodeState, positions: torch.Tensor):
    """TransformerEncoderLayer.decode_step (native/patch_encoder.py:77-85) with
    MultiHeadAttention.decode_step (native/layers.py:210-249); x [T, hidden]."""
    p = f"encoder.layers.{l}."
    H, nh, hd = cfg.hidden, cfg.heads, cfg.head_dim
    h = F.layer_norm(x, (H,), W[p + "attn_norm.weight"], W[p + "attn_norm.bias"], cfg.ln_eps)
    q = F.linear(h, W[p + "attn.q_proj.weight"]).view(-1, nh, hd).transpose(0, 1)   # [nh, T, hd]
    k = F.linear(h, W[p + "attn.k_proj.weight"]).view(-1, nh, hd).transpose(0, 1)
    v = F.linear(h, W[p + "attn.v_proj.weight"]).view(-1, nh, hd).transpose(0, 1)
    st.k[l][:, positions] = k
    st.v[l][:, positions] = v
    cap = st.k[l].shape[1]
    keys = torch.arange(cap)
    vis = (keys[None, :] <= positions[:, None]) & (keys[None, :] <= positions[-1])   # [T, cap]
    s = (q @ st.k[l].transpose(1, 2)) * hd ** -0.5
    s = s.masked_fill(~vis[None], float("-inf"))
    o = torch.softmax(s, dim=-1) @ st.v[l]                                           # [nh, T, hd]
    o = o.transpose(0, 1).reshape(-1, H)
    x = x + F.linear(o, W[p + "attn.o_proj.weight"], W[p + "attn.o_proj.bias"])
    h = F.layer_norm(x, (H,), W[p + "ffn_norm.weight"], W[p + "ffn_norm.bias"], cfg.ln_eps)
    h = F.silu(F.linear(h, W[p + "ffn.fc1.weight"], W[p + "ffn.fc1.bias"]))
    return x + F.linear(h, W[p + "ffn.fc2.weight"], W[p + "ffn.fc2.bias"])


def decode_patch(W, cfg: PatchEncConfig, patch: torch.Tensor, st: DecodeState) -> torch.Tensor:
    """VAESemanticEncoder.decode_patch for one request (native/patch_encoder.py:
    198-215) plus the caller's state update (engine.py:786-800): patch
    [P, latent_dim] -> embedding [out_dim]; st advances by out_ds_rate."""
    W = {k: v.float() for k, v in W.items()}
    x, tail = downsample_step(W, cfg, patch.float(), st.conv_tail)
    positions = torch.arange(cfg.ods) + st.seq_len
    for l in range(cfg.n_layers):
        x = layer_decode(W, cfg, l, x, st, positions)
    st.conv_tail = tail
    st.seq_len += cfg.ods
    return F.linear(x.reshape(1, -1), W["out_proj.weight"], W["out_proj.bias"])[0]


class PatchEncoderCacheRef:
    """FlashPatchEncoder's bookkeeping (flash_patch_encoder.py:43-69, 103-139):
    a decode state per cache row; decode_patch(patches [n, P, ld], rows [n])
    advances rows[i] by request i's patch and returns [n, 1, out_dim]."""

    def __init__(self, W, cfg: PatchEncConfig, max_batch: int, cap: int):
        self.W, self.cfg, self.cap = W, cfg, cap
        self.rows = [init_state(cfg, cap) for _ in range(max_batch)]

    def reset_rows(self, rows):
        for r in rows:
            self.rows[int(r)] = init_state(self.cfg, self.cap)

    def seqlen(self, r) -> int:
        return self.rows[int(r)].seq_len

    @torch.no_grad()
    def decode_patch(self, patches: torch.Tensor, rows) -> torch.Tensor:
        rows = [int(r) for r in rows]
        if len(set(rows)) != len(rows):
            raise ValueError("rows must be distinct")
        out = [decode_patch(self.W, self.cfg, patches[i], self.rows[r]) for i, r in enumerate(rows)]
        return torch.stack(out)[:, None]
