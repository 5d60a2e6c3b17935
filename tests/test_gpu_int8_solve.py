"""The W8A8 solve (the reference's quantize_dit_ DiT, D/int8_dit.py) through the
C ABI against the oracle's int8 regime: the bf16 DiT with every linear of
min(in, out) >= 512 computed as the fixture-pinned Int8DynamicLinear
restatement. GPU only.

Bar: latents after the NFE = 4 solve at per-row cosine >= 0.9999 and max |diff|
<= 0.02 * max |ref| against the int8 regime (the solve's bar); against the
float32 oracle the int8 solve is reported (the cost of W8A8 itself)."""
from __future__ import annotations

import pytest
import torch

from conftest import cos_stats
from oracle import dit_ref as R
from test_gpu_parity import FULL, _assert_latents, _cuda_bf16

pytestmark = pytest.mark.gpu

SMALL = R.DitConfig(hidden=1024, heads=16, ffn=4096, n_blocks=2, latent_dim=64, patch=16)


def _oracle(Wb, cfg, hist, noise, regime):
    dev = torch.device("cuda")
    Wd = {k: v.to(dev) for k, v in Wb.items()}
    with torch.no_grad():
        return R.meanflow_solve_varlen(Wd, cfg, [h.to(dev) for h in hist], None, noise.to(dev), 4, regime).cpu()


def _solve(head, cfg, hist, noise):
    from nanovllm_dots_amd import HipMeanflow
    inp, _, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    return mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(g),
              noise=_cuda_bf16(noise)).float().cpu()


@pytest.mark.parametrize("cfg,n,lo,hi,seed", [(SMALL, 3, 30, 200, 1), (FULL, 4, 64, 384, 2)])
def test_int8_solve_matches_int8_oracle(cfg, n, lo, hi, seed):
    from nanovllm_dots_amd import FMSpec, HipFMHead
    W = R.random_dit_weights(cfg, seed)
    Wb = R.weights_for_regime(W, "int8")
    lens, hist, noise = R.synthetic_requests(n, lo, hi, cfg, seed, regime="bf16")
    print(f"int8 solve: {cfg.n_blocks} blocks, lens {lens}", flush=True)
    head = HipFMHead(FMSpec.of(cfg), W, device="cuda", int8=True)
    assert head.int8
    got = _solve(head, cfg, hist, noise)
    ref8 = _oracle(Wb, cfg, hist, noise, "int8")
    _assert_latents(got, ref8, cfg.latent_dim, f"int8 solve vs int8 oracle ({cfg.n_blocks} blocks)")
    ref32 = _oracle(Wb, cfg, hist, noise, "fp32")
    cmin, cmean = cos_stats(got, ref32, cfg.latent_dim)
    print(f"int8 solve vs fp32 oracle: cos min {cmin:.5f} mean {cmean:.6f}", flush=True)
    assert cmin >= 0.99
    # back to bf16 on the same handle
    head.set_int8(False)
    _assert_latents(_solve(head, cfg, hist, noise), ref32, cfg.latent_dim, "bf16 solve after int8 off vs fp32")
    head.close()


def test_quantized_module_weights_are_taken_as_they_are():
    """A state dict after the reference's quantize_dit_ (Int8DynamicLinear:
    ``Wt_int8`` [in, out] + ``w_scale``, no ``weight``) runs the W8A8 solve with
    those int8 weights: bit-identical to quantising the same bf16 weights here."""
    from nanovllm_dots_amd import FMSpec, HipFMHead
    from oracle.int8_ref import quantize_weight
    cfg = SMALL
    W = R.random_dit_weights(cfg, 3)
    head_ref = HipFMHead(FMSpec.of(cfg), W, device="cuda", int8=True)
    Wq = dict(W)
    for name in head_ref.int8_linear_names():
        w = R.round_bf16(Wq.pop(name + ".weight"))
        q, sc = quantize_weight(w)
        Wq[name + ".Wt_int8"] = q.t().contiguous()
        Wq[name + ".w_scale"] = sc
    head_q = HipFMHead(FMSpec.of(cfg), Wq, device="cuda")
    assert head_q.int8
    lens, hist, noise = R.synthetic_requests(2, 20, 90, cfg, 4, regime="bf16")
    print(f"quantized module weights: lens {lens}", flush=True)
    a, b = _solve(head_ref, cfg, hist, noise), _solve(head_q, cfg, hist, noise)
    assert torch.equal(a, b)
    partial = dict(Wq)
    name = head_ref.int8_linear_names()[5]
    partial[name + ".weight"] = W[name + ".weight"]
    del partial[name + ".Wt_int8"], partial[name + ".w_scale"]
    with pytest.raises(RuntimeError, match="partly quantised"):
        HipFMHead(FMSpec.of(cfg), partial, device="cuda")
    head_ref.close()
    head_q.close()


def test_fused_layernorm_quantiser_is_bit_identical():
    """QKV's and fc1's input rows quantised inside LayerNorm+modulate against the
    separate per-token quantiser pass over the bf16 rows: the same int8 rows and
    scales, so the same latents bit for bit (solve with its latent tail, and
    the cached solve's prime and decode passes)."""
    from nanovllm_dots_amd import FMSpec, HipFMCache, HipFMHead
    cfg = SMALL
    W = R.random_dit_weights(cfg, 5)
    head = HipFMHead(FMSpec.of(cfg), W, device="cuda", int8=True)
    lens, hist, noise = R.synthetic_requests(3, 25, 160, cfg, 6, regime="bf16")
    print(f"fused ln quantiser: lens {lens}", flush=True)
    outs = []
    for fused in (True, False):
        head.set_ln_quant(fused)
        solve = _solve(head, cfg, hist, noise)
        cache = HipFMCache(head, 3, max(lens) + 24, 4)
        prefix = [h[:-1] for h in hist]
        rows = torch.zeros(3, max(p.shape[0] for p in prefix), cfg.hidden)
        for i, p in enumerate(prefix):
            rows[i, :p.shape[0]] = p
        cache.extend(rows.cuda(), [p.shape[0] for p in prefix])
        cached = cache.solve(torch.stack([h[-1] for h in hist]).cuda(), noise=noise.cuda())
        cache.close()
        outs.append((solve, cached))
    head.set_ln_quant(True)
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    head.close()
