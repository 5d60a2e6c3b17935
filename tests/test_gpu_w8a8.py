"""W8A8 path vs torch._int_mm, the oracle and the reference-generated fixture.
GPU only. Bar: int32 accumulators, int8 operands and scales bit-exact; the bf16
dequantised output bit-exact against the oracle's op order (int8_dit.py:60-65)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import int8_ref as Q
from oracle.dit_ref import round_bf16

pytestmark = pytest.mark.gpu


def _bits(a):
    return torch.from_numpy(a).view(torch.bfloat16)


def test_golden_int8_linear_bit_exact():
    """The reference Int8DynamicLinear output (fixture) from HipInt8Linear."""
    from nanovllm_dots_amd.int8 import HipInt8Linear
    g = load_golden("int8_linear.npz")
    W, b, x = _bits(g["W_bf16bits"]), _bits(g["b_bf16bits"]), _bits(g["x_bf16bits"])
    lin = torch.nn.Linear(W.shape[1], W.shape[0]).to(device="cuda", dtype=torch.bfloat16)
    lin.weight.data = W.cuda()
    lin.bias.data = b.cuda()
    m = HipInt8Linear(lin)
    assert torch.equal(m.W_int8.t().contiguous().cpu(), torch.from_numpy(g["Wt_int8"]))
    assert torch.equal(m.w_scale.cpu(), torch.from_numpy(g["w_scale"]))
    y = m(x.cuda()).cpu()
    ref = _bits(g["y_bf16bits"])
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), (y.float() - ref.float()).abs().max()


@pytest.mark.parametrize("M,K", [(37, 1024), (513, 4096), (4096, 1024), (5, 2048), (61, 2056), (9, 8)])
def test_activation_quant_bit_exact(M, K):
    from nanovllm_dots_amd.int8 import quant_act
    rs = np.random.RandomState(M + K)
    x = torch.from_numpy(rs.standard_normal((M, K)).astype(np.float32)).bfloat16()
    x[0] = 0
    x[1] *= 1e-3
    q, s = quant_act(x.cuda())
    qr, sr = Q.quantize_act(x.float())
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr)


def test_weight_quant_bit_exact():
    from nanovllm_dots_amd.int8 import quant_weight
    rs = np.random.RandomState(3)
    W = torch.from_numpy((0.02 * rs.standard_normal((1024, 4096))).astype(np.float32)).bfloat16()
    W[5] = 0
    q, s = quant_weight(W.cuda())
    qr, sr = Q.quantize_weight(W.float())
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr)


C4_KN = [(1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024)]


@pytest.mark.parametrize("K,N", C4_KN)
@pytest.mark.parametrize("M", [4096, 333])
def test_int32_accumulators_match_int_mm(M, K, N):
    """The W8A8 configuration's (K, N) shapes; int32 == torch._int_mm exactly."""
    from nanovllm_dots_amd.int8 import gemm_w8a8
    g = torch.Generator(device="cpu").manual_seed(M + K + N)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).cuda()
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    print(f"w8a8 int32 M={M} K={K} N={N}", flush=True)
    acc = gemm_w8a8(xq, wq, out_int32=True)
    ref = torch._int_mm(xq, wq.t().contiguous())
    assert torch.equal(acc, ref)


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 5, 7, 8, 9, 10, 11])
def test_int32_all_tiles(tile):
    from nanovllm_dots_amd.int8 import gemm_w8a8
    M, K, N = 700, 1024, 1024
    g = torch.Generator(device="cpu").manual_seed(tile)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).cuda()
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    acc = gemm_w8a8(xq, wq, out_int32=True, tile=tile)
    assert torch.equal(acc, torch._int_mm(xq, wq.t().contiguous()))


def test_extreme_values_no_overflow():
    """|acc| <= K * 127^2 < 2^31 at K = 4096: all-(+-127) operands."""
    from nanovllm_dots_amd.int8 import gemm_w8a8
    M, K, N = 256, 4096, 256
    xq = torch.full((M, K), 127, dtype=torch.int8, device="cuda")
    xq[::2] = -127
    wq = torch.full((N, K), -127, dtype=torch.int8, device="cuda")
    acc = gemm_w8a8(xq, wq, out_int32=True)
    assert torch.equal(acc, torch._int_mm(xq, wq.t().contiguous()))
    assert acc.abs().max().item() == K * 127 * 127


@pytest.mark.parametrize("K,N", C4_KN)
def test_dequant_linear_matches_oracle(K, N):
    """HipInt8Linear vs the oracle's Int8DynamicLinear restatement, bit-exact."""
    from nanovllm_dots_amd.int8 import HipInt8Linear
    M = 1000
    rs = np.random.RandomState(K * 7 + N)
    lin = torch.nn.Linear(K, N)
    lin.weight.data = torch.from_numpy((0.02 * rs.standard_normal((N, K))).astype(np.float32))
    lin.bias.data = torch.from_numpy((0.02 * rs.standard_normal((N,))).astype(np.float32))
    lin = lin.to(device="cuda", dtype=torch.bfloat16)
    x = torch.from_numpy(rs.standard_normal((M, K)).astype(np.float32)).bfloat16()
    y = HipInt8Linear(lin)(x.cuda()).float().cpu()
    Wq, sw = Q.quantize_weight(lin.weight.detach().float().cpu())
    ref, _, _, _ = Q.int8_linear(x.float(), Wq, sw, lin.bias.detach().float().cpu())
    assert torch.equal(y, ref), (y - ref).abs().max()
    # quality vs the bf16 linear (the reference measured ~1 % relative error)
    bf = (x.float() @ lin.weight.detach().float().cpu().t() + lin.bias.detach().float().cpu())
    rel = ((y - bf).norm() / bf.norm()).item()
    assert rel < 0.03, rel


def test_quantize_dit_swaps_eligible_linears():
    from nanovllm_dots_amd.int8 import HipInt8Linear, quantize_dit_
    net = torch.nn.Sequential(torch.nn.Linear(1024, 1024), torch.nn.SiLU(), torch.nn.Linear(1024, 64))
    net = net.to(device="cuda", dtype=torch.bfloat16)
    assert quantize_dit_(net) == 1
    assert isinstance(net[0], HipInt8Linear) and isinstance(net[2], torch.nn.Linear)
    out = net(torch.randn(20, 1024, device="cuda", dtype=torch.bfloat16))
    assert out.shape == (20, 64) and torch.isfinite(out.float()).all()


def _split_ws():
    # one 256x256 f32 partial tile + one counter per CU (256 CUs); zero-filled before first use
    return torch.zeros((1 << 26) + (1 << 16), dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("M,K,N,tile", [(36937, 4096, 1024, 8), (36937, 1024, 4096, 8), (20000, 4096, 1024, 0),
                                        (3000, 2048, 256, 3), (36937, 4096, 1024, 9), (36937, 1024, 4096, 9),
                                        (68, 4096, 1024, 10), (68, 1024, 3072, 11), (100, 2048, 256, 10)])
def test_int32_ksplit_exact(M, K, N, tile):
    """K-split of the last partial tile round: int32 partial sums add exactly."""
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    g = torch.Generator(device="cpu").manual_seed(M + K)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).cuda()
    wq = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    ws = _split_ws()
    out = torch.empty((M, N), device="cuda", dtype=torch.int32)
    print(f"w8a8 ksplit M={M} K={K} N={N} tile={tile}", flush=True)
    _lib.check(lib.dfh_gemm_w8a8_ws(_lib.ptr(xq), K, _lib.ptr(wq), K, _lib.ptr(out), N, None, None, None, M, N, K,
                                    1, tile, _lib.ptr(ws), ws.numel(), _lib.stream_ptr()), "dfh_gemm_w8a8_ws")
    ref = torch._int_mm(xq, wq.t().contiguous())
    bad = (out != ref).nonzero()
    assert bad.numel() == 0, f"{bad.shape[0]} mismatches, first rows {bad[:4].tolist()}"
