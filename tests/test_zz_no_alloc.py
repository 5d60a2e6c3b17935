"""dfh_paged_attention_noalloc (static device scratch, no allocation) against
dfh_paged_attention (caller's workspace) through the C ABI: two calls in a row,
the second smaller, bit-identical outputs (same kernels, same work split); and
a call whose workspace exceeds the static maximum is refused before any launch.
GPU only."""
from __future__ import annotations

import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _decode_case(B, L, lq, seed, H=12, Hkv=2, hd=128, bs=256):
    g = torch.Generator(device="cuda").manual_seed(seed)
    pages = B * ((L + bs - 1) // bs)
    kc = torch.randn(pages, bs, Hkv, hd, device="cuda", generator=g).bfloat16()
    vc = torch.randn(pages, bs, Hkv, hd, device="cuda", generator=g).bfloat16()
    bt = torch.randperm(pages, device="cuda", generator=g).to(torch.int32).view(B, -1).contiguous()
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    q = torch.randn(B * lq, H, hd, device="cuda", generator=g).bfloat16()
    cu_q = torch.arange(0, (B + 1) * lq, lq, dtype=torch.int32, device="cuda")
    return dict(kc=kc, vc=vc, bt=bt, lens=lens, q=q, cu_q=cu_q, B=B, L=L, lq=lq, H=H, Hkv=Hkv, hd=hd, bs=bs)


def _args(c, out):
    from nanovllm_dots_amd import _lib
    return _lib.DfhPagedAttnArgs(
        batch=c["B"], num_heads=c["H"], num_kv_heads=c["Hkv"], head_dim=c["hd"], max_seqlen_q=c["lq"],
        max_seqlen_k=c["bt"].shape[1] * c["bs"], q=_lib.ptr(c["q"]), q_stride=c["H"] * c["hd"],
        cu_seqlens_q=_lib.ptr(c["cu_q"]), k=_lib.ptr(c["kc"]), v=_lib.ptr(c["vc"]), kv_stride=c["Hkv"] * c["hd"],
        cu_seqlens_k=None, seqlens_k=_lib.ptr(c["lens"]), block_table=_lib.ptr(c["bt"]),
        block_table_stride=c["bt"].shape[1], block_size=c["bs"], out=_lib.ptr(out),
        out_stride=c["H"] * c["hd"], softmax_scale=c["hd"] ** -0.5, causal=1, workspace=None, workspace_bytes=0,
        total_q=c["q"].shape[0])


def test_noalloc_matches_workspace_entry_point_twice():
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    for B, L, lq, seed in ((64, 4096, 1, 0), (8, 1000, 4, 1)):   # the second call smaller
        c = _decode_case(B, L, lq, seed)
        ref = torch.empty_like(c["q"])
        got = torch.full_like(c["q"], float("nan"))
        a = _args(c, ref)
        need = lib.dfh_paged_attention_workspace(C.byref(a))
        ws = torch.empty((need + 3) // 4, device="cuda", dtype=torch.float32)
        a.workspace, a.workspace_bytes = _lib.ptr(ws), ws.numel() * 4
        print(f"no-alloc paged attention: B={B} L={L} lq={lq} workspace {need / 2**20:.2f} MiB", flush=True)
        _lib.check(lib.dfh_paged_attention(C.byref(a), _lib.stream_ptr()), "dfh_paged_attention")
        b = _args(c, got)
        _lib.check(lib.dfh_paged_attention_noalloc(C.byref(b), _lib.stream_ptr()), "dfh_paged_attention_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


def test_noalloc_refuses_more_than_its_scratch():
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    c = _decode_case(4, 256, 1, 2)
    out = torch.empty_like(c["q"])
    a = _args(c, out)
    a.batch, a.max_seqlen_k, a.total_q = 512, 4096, 512   # sizes only: refused before any launch
    assert lib.dfh_paged_attention_workspace(C.byref(a)) > 64 << 20
    assert lib.dfh_paged_attention_noalloc(C.byref(a), _lib.stream_ptr()) != 0
    assert b"static" in lib.dfh_last_error()
