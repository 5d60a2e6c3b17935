"""W8A8 DiT linears on gfx950 i8 MFMA (drop-in for the reference's int8 path).

``HipInt8Linear`` mirrors ``Int8DynamicLinear``
(nanovllm_dots/models/dots/int8_dit.py:34-65): per-output-channel int8 weights
quantised once in float32, per-token dynamic int8 activations quantised in the
input's dtype (bf16), int32 accumulation, then ``((acc * s_x) * s_w) + bias``.
Here the activation quantisation is one kernel and the GEMM carries the dequant
and bias in its epilogue (the reference runs them as separate torch ops around
``torch._int_mm``). The int32 accumulators are bit-identical to
``torch._int_mm``; the bf16 output follows the reference's op order and
rounding.

``quantize_dit_(dit)`` swaps eligible ``nn.Linear`` layers like the reference's
``quantize_dit_`` (int8_dit.py:71-85).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib


def quant_act(x: torch.Tensor):
    """bf16 [M, K] -> (q int8 [M, K], scale f32 [M])."""
    lib = _lib.lib()
    x = x.to(torch.bfloat16).contiguous()
    M, K = x.shape
    q = torch.empty((M, K), device=x.device, dtype=torch.int8)
    s = torch.empty((M,), device=x.device, dtype=torch.float32)
    _lib.check(lib.dfh_quant_act_i8(_lib.ptr(x), K, _lib.ptr(q), K, _lib.ptr(s), M, K, _lib.stream_ptr()),
               "dfh_quant_act_i8")
    return q, s


def quant_weight(w: torch.Tensor):
    """bf16 [N, K] -> (q int8 [N, K], scale f32 [N])."""
    lib = _lib.lib()
    w = w.to(torch.bfloat16).contiguous()
    N, K = w.shape
    q = torch.empty((N, K), device=w.device, dtype=torch.int8)
    s = torch.empty((N,), device=w.device, dtype=torch.float32)
    _lib.check(lib.dfh_quant_weight_i8(_lib.ptr(w), _lib.ptr(q), _lib.ptr(s), N, K, _lib.stream_ptr()),
               "dfh_quant_weight_i8")
    return q, s


def gemm_w8a8(xq: torch.Tensor, wq: torch.Tensor, sx=None, sw=None, bias=None, *, out_int32=False,
              tile: int = -1):
    """int8 [M, K] x int8 [N, K]^T -> int32 [M, N] (out_int32) or dequantised bf16."""
    lib = _lib.lib()
    M, K = xq.shape
    N = wq.shape[0]
    if wq.shape[1] != K:
        raise RuntimeError(f"K mismatch {tuple(xq.shape)} x {tuple(wq.shape)}")
    out = torch.empty((M, N), device=xq.device, dtype=torch.int32 if out_int32 else torch.bfloat16)
    b = bias.to(torch.bfloat16).contiguous() if bias is not None else None
    _lib.check(lib.dfh_gemm_w8a8(_lib.ptr(xq), xq.stride(0), _lib.ptr(wq), wq.stride(0), _lib.ptr(out), N,
                                 _lib.ptr(sx), _lib.ptr(sw), _lib.ptr(b), M, N, K, int(out_int32), tile,
                                 _lib.stream_ptr()), "dfh_gemm_w8a8")
    return out


class HipInt8Linear(nn.Module):
    """Drop-in for nn.Linear / Int8DynamicLinear: int8 weight (per-out-channel)
    x int8 activation (per-token, dynamic), dequantised back to bf16."""

    def __init__(self, lin: nn.Linear):
        super().__init__()
        q, s = quant_weight(lin.weight.data)
        self.register_buffer("W_int8", q)          # [out, in]
        self.register_buffer("w_scale", s)         # [out]
        self.bias = lin.bias
        self.in_features = lin.in_features
        self.out_features = lin.out_features

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        xq, sx = quant_act(x2)
        out = gemm_w8a8(xq, self.W_int8, sx, self.w_scale, self.bias)
        return out.to(x.dtype).reshape(*shape[:-1], self.out_features)


def quantize_dit_(dit, *, min_features: int = 512) -> int:
    """W8A8 every plain nn.Linear of ``dit`` whose smaller side has at least
    ``min_features`` features (the eligibility rule of int8_dit.py:71-85), in
    place; returns how many were replaced. ``HipFMHead`` takes such a module's
    int8 weights as they are (its W8A8 solve)."""
    targets = [(parent, name, child) for parent in dit.modules() for name, child in parent.named_children()
               if type(child) is nn.Linear and min(child.in_features, child.out_features) >= min_features]
    for parent, name, child in targets:
        setattr(parent, name, HipInt8Linear(child))
    return len(targets)
