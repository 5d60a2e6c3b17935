"""The oracle's int8 regime (the bf16 DiT after quantize_dit_): its W8A8 linear
is the fixture-pinned Int8DynamicLinear restatement, and only the linears with
min(in, out) >= 512 take it. CPU."""
from __future__ import annotations

import numpy as np
import torch

from conftest import load_golden
from oracle import dit_ref as R
from oracle import int8_ref as I


def test_int8_regime_linear_is_the_pinned_w8a8_linear():
    """The regime's float64 product path gives the reference fixture's bf16
    output bit for bit (int8_linear.npz, written by Int8DynamicLinear)."""
    g = load_golden("int8_linear.npz")
    W = torch.from_numpy(g["W_bf16bits"]).view(torch.bfloat16).float()
    b = torch.from_numpy(g["b_bf16bits"]).view(torch.bfloat16).float()
    x = torch.from_numpy(g["x_bf16bits"]).view(torch.bfloat16).float()
    want = torch.from_numpy(g["y_bf16bits"]).view(torch.bfloat16).float()
    Rg = R._R("int8")
    Rg.INT8_MIN_FEATURES = 128          # the fixture's layer is 128 x 192
    got = Rg.linear(x, W, b)
    assert torch.equal(got, want)
    ref, *_ = I.int8_linear(x, *I.quantize_weight(W), b)
    assert torch.equal(got, ref)


def test_int8_regime_only_touches_eligible_linears():
    rs = np.random.RandomState(0)
    x = R.round_bf16(torch.from_numpy(rs.standard_normal((9, 256)).astype(np.float32)))
    small = R.round_bf16(torch.from_numpy((0.02 * rs.standard_normal((1024, 256))).astype(np.float32)))
    big = R.round_bf16(torch.from_numpy((0.02 * rs.standard_normal((1024, 512))).astype(np.float32)))
    x2 = R.round_bf16(torch.from_numpy(rs.standard_normal((9, 512)).astype(np.float32)))
    assert torch.equal(R._R("int8").linear(x, small), R._R("bf16").linear(x, small))   # min 256 < 512
    q, d = R._R("int8").linear(x2, big), R._R("bf16").linear(x2, big)
    assert not torch.equal(q, d)
    assert torch.nn.functional.cosine_similarity(q.flatten(), d.flatten(), dim=0) > 0.999
