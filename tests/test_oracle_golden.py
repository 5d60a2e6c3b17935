"""The oracle against fixtures written by the reference's own DiT / mask
builders / W8A8 linear (tests/golden/gen_golden.py). CPU only."""
from __future__ import annotations

import ast

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import dit_ref as R
from oracle import int8_ref as Q

TINY = ["tiny_rope.npz", "tiny_qknorm_bias.npz", "tiny_rms_norope.npz"]


def _case(name):
    g = load_golden(name)
    cfg = R.DitConfig(**ast.literal_eval(str(g["cfg"])))
    W = R.random_dit_weights(cfg, int(g["seed"]))
    return g, cfg, W


@pytest.mark.parametrize("name", TINY)
def test_mask_and_pos_match_reference_builders(name):
    g, cfg, _ = _case(name)
    lens = [int(x) for x in g["lens"]]
    T = g["mask"].shape[-1]
    for i, L in enumerate(lens):
        assert np.array_equal(R.build_fm_attn_mask(L, T, cfg.patch).numpy(), g["mask"][i])
        assert np.array_equal(R.build_fm_pos_ids(L, T, cfg.patch).numpy(), g["pos"][i])


@pytest.mark.parametrize("name", TINY)
def test_dit_forward_matches_reference(name):
    g, cfg, W = _case(name)
    t = lambda k: torch.from_numpy(g[k])
    out = R.dit_forward(W, cfg, t("x"), t("t"), t("dur") if cfg.meanflow else None,
                        t("mask"), t("pos"), t("g"), regime="fp32")
    ref = t("dit_out")
    assert out.shape == ref.shape
    err = (out - ref).abs().max().item()
    assert err < 2e-5 * max(1.0, ref.abs().max().item()), err


@pytest.mark.parametrize("name", ["tiny_rope.npz", "tiny_qknorm_bias.npz", "tiny_rms_norope.npz"])
def test_meanflow_matches_reference_loop(name):
    g, cfg, W = _case(name)
    t = lambda k: torch.from_numpy(g[k])
    z = R.meanflow_solve(W, cfg, t("inp"), t("mask"), t("pos"), t("g"), t("noise"),
                         num_steps=4, regime="fp32")
    ref = t("mf_out")
    err = (z - ref).abs().max().item()
    assert err < 5e-5 * max(1.0, ref.abs().max().item()), err


@pytest.mark.parametrize("name", TINY)
def test_varlen_twin_equals_padded_reference(name):
    """Packed rows + implicit mask == the reference's padded dense-mask output
    on every valid row (padding rows dropped)."""
    g, cfg, W = _case(name)
    lens = [int(x) for x in g["lens"]]
    x = torch.from_numpy(g["x"])
    T, P = x.shape[1], cfg.patch
    rows = [torch.cat([x[i, :L], x[i, T - P:]]) for i, L in enumerate(lens)]
    out = R.dit_forward_varlen(W, cfg, torch.cat(rows), lens, torch.from_numpy(g["t"]),
                               torch.from_numpy(g["dur"]) if cfg.meanflow else None,
                               torch.from_numpy(g["g"]), regime="fp32")
    ref = torch.from_numpy(g["dit_out"])
    off = 0
    for i, L in enumerate(lens):
        want = torch.cat([ref[i, :L], ref[i, T - P:]])
        got = out[off:off + L + P]
        assert (got - want).abs().max().item() < 2e-5
        off += L + P


def test_one_block_80_rows_matches_reference():
    g = load_golden("c1_block.npz")
    cfg = R.DitConfig(**ast.literal_eval(str(g["cfg"])))
    W = R.random_dit_weights(cfg, 0)
    rs = np.random.RandomState(0)
    x = torch.from_numpy(rs.standard_normal((1, 80, 1024)).astype(np.float32))
    mask = R.build_fm_attn_mask(64, 80, 16)[None]
    pos = R.build_fm_pos_ids(64, 80, 16)[None]
    t = torch.full((1,), 0.25)
    out, h = R.dit_forward(W, cfg, x, t, t, mask, pos, torch.zeros(1, 1024), regime="fp32",
                           return_hidden=True)
    rows = [int(r) for r in g["rows"]]
    assert torch.allclose(h[0, rows], torch.from_numpy(g["block_rows"]), atol=2e-4, rtol=1e-4)
    assert abs(h.double().sum().item() - float(g["block_sum"])) < 1e-2
    assert abs((h.double() ** 2).sum().item() / float(g["block_sumsq"]) - 1) < 1e-5
    assert torch.allclose(out, torch.from_numpy(g["out"]), atol=2e-5, rtol=1e-4)


def _bits(a):
    return torch.from_numpy(a).view(torch.bfloat16).float()


def test_int8_weight_quant_matches_reference():
    g = load_golden("int8_linear.npz")
    Wq, s_w = Q.quantize_weight(_bits(g["W_bf16bits"]))
    assert np.array_equal(Wq.t().contiguous().numpy(), g["Wt_int8"])
    assert np.array_equal(s_w.numpy(), g["w_scale"])


def test_int8_linear_matches_reference_bit_exact():
    g = load_golden("int8_linear.npz")
    Wq, s_w = Q.quantize_weight(_bits(g["W_bf16bits"]))
    y, acc, q, s = Q.int8_linear(_bits(g["x_bf16bits"]), Wq, s_w, _bits(g["b_bf16bits"]))
    ref = _bits(g["y_bf16bits"])
    assert torch.equal(y, ref), (y - ref).abs().max()
    # library check of the exact int64 brute force
    assert torch.equal(acc, torch._int_mm(q, Wq.t().contiguous()))
