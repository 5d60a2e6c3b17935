"""W8A8 DiT linear restated from D/int8_dit.py (test infrastructure only).

``D/`` = ``nanovllm_dots/models/dots/``. The activation quantisation runs in the
input's dtype (bf16): each bf16 op is one float32 operation followed by a
round-to-nearest-even to bf16, which is how torch evaluates bf16 tensors. The
integer product is brute-forced in int64 numpy (exact) — ``torch._int_mm`` is
the library check in the tests.
"""
from __future__ import annotations

import numpy as np
import torch

from .dit_ref import round_bf16


def quantize_weight(W: torch.Tensor):
    """Int8DynamicLinear.__init__ (D/int8_dit.py:40-45): float32 math,
    s_w = max(amax_row(|W|)/127, 1e-8), Wq = clamp(round(W/s_w), -127, 127).
    Returns (Wq [out, in] int8, s_w [out] float32)."""
    Wf = W.float()
    s_w = (Wf.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=1e-8)
    Wq = torch.round(Wf / s_w).clamp(-127, 127).to(torch.int8)
    return Wq, s_w.squeeze(1)


def quantize_act(x_bf16_values: torch.Tensor):
    """Int8DynamicLinear.forward activation quant (D/int8_dit.py:57-58) for a bf16
    input given as float32 values, [M, K]:
      amax = max|x| (exact in bf16);  s = bf16(amax / 127);  s = max(s, bf16(1e-8))
      q = clamp(round_half_even(bf16(x / s)), -127, 127).
    Returns (q int8 [M, K], s float32 [M] holding bf16 values)."""
    x = x_bf16_values.float()
    amax = x.abs().amax(dim=1, keepdim=True)
    s = round_bf16(amax / 127.0)
    s = torch.maximum(s, round_bf16(torch.tensor(1e-8)))
    q = round_bf16(x / s)
    q = torch.round(q).clamp(-127, 127).to(torch.int8)   # torch.round is half-to-even
    return q, s.squeeze(1)


def int_mm_exact(xq: torch.Tensor, Wq: torch.Tensor) -> torch.Tensor:
    """int32 accumulators of xq [M,K] @ Wq[N,K]^T computed exactly in int64."""
    a = xq.numpy().astype(np.int64)
    b = Wq.numpy().astype(np.int64)
    acc = a @ b.T
    assert np.abs(acc).max(initial=0) < 2 ** 31
    return torch.from_numpy(acc.astype(np.int32))


def dequant(acc: torch.Tensor, s_x: torch.Tensor, s_w: torch.Tensor, bias):
    """D/int8_dit.py:60-65: ((acc.f32 * s_x) * s_w) + bias.f32 -> bf16 (as
    float32 values); each product and the sum rounded to float32 separately."""
    out = acc.float() * s_x.float()[:, None]
    out = out * s_w[None, :]
    if bias is not None:
        out = out + bias.float()[None, :]
    return round_bf16(out)


def int8_linear(x_bf16_values: torch.Tensor, Wq: torch.Tensor, s_w: torch.Tensor, bias):
    """Int8DynamicLinear.forward (D/int8_dit.py:50-65) for M >= 17 rows; the
    reference pads M < 17 with zero rows whose outputs it drops, which leaves the
    kept rows unchanged."""
    q, s = quantize_act(x_bf16_values)
    acc = int_mm_exact(q, Wq)
    return dequant(acc, s, s_w, bias), acc, q, s
