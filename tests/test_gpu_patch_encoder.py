"""The patch encoder's batched per-patch decode (HipPatchEncoder, the
FlashPatchEncoder drop-in) against the float32 oracle that the reference's own
patch encoder pins (tests/golden/patch_encoder.npz). GPU only.

Size: the SuperviseEncoder defaults (hidden 1024, 16 heads x 64, MLP 4096,
6 layers), latent patches of 16 x 64, out_dim 1536 (Qwen2-1.5B width). The HIP
path holds the parameters in bf16 (as the reference loads them); the oracle runs
float32 on the same bf16-valued parameters and patches.

Bar (per request embedding): cosine >= 0.9999 and max |diff| <= 0.02 * max |ref|
-- the solve's latent bar; the reference's own flash-vs-SDPA check is 0.999
(tests/test_patch_encoder.py:54)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import patch_encoder_ref as PE
from oracle.dit_ref import round_bf16

pytestmark = pytest.mark.gpu

COS = 0.9999
MAXABS_FRAC = 0.02


def _setup(max_batch, cap, seed=0, cfg=None):
    from nanovllm_dots_amd import HipPatchEncoder
    cfg = cfg or PE.PatchEncConfig()
    W = {k: round_bf16(v) for k, v in PE.random_pe_weights(cfg, seed).items()}
    dims = dict(latent_dim=cfg.latent_dim, patch=cfg.patch, hidden=cfg.hidden, heads=cfg.heads, ffn=cfg.ffn,
                n_layers=cfg.n_layers, out_dim=cfg.out_dim, ln_eps=cfg.ln_eps)
    hip = HipPatchEncoder(max_batch=max_batch, max_seq_len=cap, device="cuda", weights=W, dims=dims)
    ref = PE.PatchEncoderCacheRef(W, cfg, max_batch, cap)
    return cfg, hip, ref


def _check(got, ref, label):
    got, ref = got.float().cpu().reshape(ref.shape[0], -1), ref.float().reshape(ref.shape[0], -1)
    cos = torch.nn.functional.cosine_similarity(got, ref, dim=-1)
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    print(f"{label}: cos min {cos.min().item():.6f} maxabs {err:.4g} (|ref| {scale:.3g})", flush=True)
    assert cos.min().item() >= COS, label
    assert err <= MAXABS_FRAC * scale, label


def test_decode_rows_at_different_lengths_match_oracle():
    """Shuffled subsets of 6 cache rows per call, so the requests of one call
    are at different history lengths (the continuous-batching case of
    flash_patch_encoder.py:103-139); lengths advance by 8 tokens per patch."""
    cfg, hip, ref = _setup(max_batch=6, cap=512)
    rs = np.random.RandomState(11)
    plan = [[5, 0, 3], [0, 1, 2, 3, 4, 5], [2], [4, 2, 0], [1, 5, 3, 0], [3, 2]]
    for step, rows in enumerate(plan):
        patches = round_bf16(torch.from_numpy(rs.standard_normal((len(rows), cfg.patch, cfg.latent_dim))
                                              .astype(np.float32)))
        print(f"patch encoder step {step}: rows {rows}", flush=True)
        got = hip.decode_patch(patches.cuda(), torch.tensor(rows, dtype=torch.int32).cuda())
        want = ref.decode_patch(patches, rows)
        assert got.shape == (len(rows), 1, cfg.out_dim)
        _check(got, want, f"step {step} rows {rows}")
    lens, overflow = hip.lengths()
    assert lens == [ref.seqlen(r) for r in range(6)] and not overflow
    hip.close()


def test_reset_rows_and_capacity_overflow_flag():
    """reset_rows starts a row afresh (its next decode equals a new request's);
    a row decoded past its capacity appends nothing, stays in bounds and
    raises the overflow flag that lengths() reports."""
    cfg = PE.PatchEncConfig(n_layers=2)
    cfg_, hip, ref = _setup(max_batch=2, cap=256, seed=1, cfg=cfg)   # 256 tokens = 32 patches per row
    rs = np.random.RandomState(12)
    mk = lambda k: round_bf16(torch.from_numpy(rs.standard_normal((k, cfg.patch, cfg.latent_dim)).astype(np.float32)))
    for _ in range(3):
        p = mk(2)
        hip.decode_patch(p.cuda(), [0, 1])
        ref.decode_patch(p, [0, 1])
    hip.reset_rows([1])
    ref.reset_rows([1])
    p = mk(2)
    print("patch encoder: after reset of row 1", flush=True)
    _check(hip.decode_patch(p.cuda(), [1, 0]), ref.decode_patch(p, [1, 0]), "after reset")
    lens, overflow = hip.lengths()
    assert lens == [32, 8] and not overflow
    # row 1 to its capacity (256 tokens), then one patch more
    for _ in range(31):
        hip.decode_patch(mk(1).cuda(), [1])
    lens, overflow = hip.lengths()
    assert lens[1] == 256 and not overflow
    out = hip.decode_patch(mk(1).cuda(), [1])
    lens, overflow = hip.lengths()
    print(f"past capacity: lengths {lens}, overflow {overflow}", flush=True)
    assert overflow and lens[1] == 256 and torch.isfinite(out.float()).all()
    hip.close()


def test_rejected_inputs():
    from nanovllm_dots_amd import HipPatchEncoder
    cfg = PE.PatchEncConfig(n_layers=1)
    W = {k: round_bf16(v) for k, v in PE.random_pe_weights(cfg, 0).items()}
    dims = dict(latent_dim=cfg.latent_dim, patch=cfg.patch, hidden=cfg.hidden, heads=cfg.heads, ffn=cfg.ffn,
                n_layers=cfg.n_layers, out_dim=cfg.out_dim)
    with pytest.raises(RuntimeError, match="hidden"):
        HipPatchEncoder(max_batch=2, max_seq_len=256, device="cuda", weights=W, dims=dict(dims, hidden=1000))
    hip = HipPatchEncoder(max_batch=2, max_seq_len=256, device="cuda", weights=W, dims=dims)
    with pytest.raises(RuntimeError, match="requests"):
        hip.decode_patch(torch.zeros(3, cfg.patch, cfg.latent_dim, device="cuda"), [0, 1, 1])
    with pytest.raises(RuntimeError, match="expected"):
        hip.decode_patch(torch.zeros(1, cfg.patch + 2, cfg.latent_dim, device="cuda"), [0])
    hip.close()
