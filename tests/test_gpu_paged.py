"""Paged KV cache of the LLM backbone on the GPU (store_kvcache, paged /
varlen attention) against the float64 oracle. GPU only.

Bar: store_kvcache bit-exact; attention outputs (bf16) within 1e-2 + 2^-8 |ref|
of the float64 oracle on the same bf16 inputs (the bf16 output rounding is up to
2^-9 |ref|, and P enters the P.V product in bf16), and per-row cosine >= 0.99999."""
from __future__ import annotations

import pytest
import torch

from oracle import paged_attn_ref as P

pytestmark = pytest.mark.gpu

ATOL = 1e-2
RTOL = 2.0 ** -8
COS = 0.99999


def _bf(x):
    return x.to(device="cuda", dtype=torch.bfloat16).contiguous()


def _check(got, ref, label):
    got = got.float().cpu().double()
    diff = (got - ref).abs()
    err = diff.max().item()
    excess = (diff - (ATOL + RTOL * ref.abs())).max().item()
    c = torch.nn.functional.cosine_similarity(got.reshape(-1, got.shape[-1]), ref.reshape(-1, ref.shape[-1]), dim=-1)
    print(f"{label}: max abs {err:.3g}, cos min {c.min().item():.7f}", flush=True)
    assert excess <= 0, f"{label}: {excess:.3g} over the bar"
    assert c.min().item() >= COS, label


def _paged(lens, Hkv, hd, bs, seed, spare_pages=3):
    """Random K/V per sequence scattered into shuffled pages of a paged cache."""
    g = torch.Generator().manual_seed(seed)
    n_pages = sum((L + bs - 1) // bs for L in lens) + spare_pages
    perm = torch.randperm(n_pages, generator=g).tolist()
    kc = torch.randn(n_pages, bs, Hkv, hd, generator=g)
    vc = torch.randn(n_pages, bs, Hkv, hd, generator=g)
    width = max((L + bs - 1) // bs for L in lens) + 1
    tables, nxt = [], 0
    for L in lens:
        npg = (L + bs - 1) // bs
        tables.append(perm[nxt:nxt + npg] + [-1] * (width - npg))
        nxt += npg
    return _bf(kc), _bf(vc), torch.tensor(tables, dtype=torch.int32)


def _cu(lens):
    return torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)


# GQA groups 6, 1, 4, 4, 16 and 40: a decode row tile holds 32 (token, head) rows,
# so the last two fill half a tile and two tiles (32 + 8 rows)
@pytest.mark.parametrize("H,Hkv,hd", [(12, 2, 128), (16, 16, 64), (8, 2, 64), (12, 3, 128), (32, 2, 128),
                                      (40, 1, 64)])
def test_decode_paged_matches_oracle(H, Hkv, hd):
    from nanovllm_dots_amd.paged_attention import flash_attn_with_kvcache
    lens = [1, 255, 256, 257, 700, 1500, 3001]
    bs = 256
    print(f"decode H={H} Hkv={Hkv} hd={hd} lens={lens}", flush=True)
    kc, vc, bt = _paged(lens, Hkv, hd, bs, seed=H + hd)
    B = len(lens)
    q = _bf(torch.randn(B, 1, H, hd, generator=torch.Generator().manual_seed(1)))
    out = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor(lens, dtype=torch.int32).cuda(),
                                  block_table=bt.cuda(), softmax_scale=hd ** -0.5, causal=True)
    ref = P.attention(q.view(B, H, hd).cpu(), kc.cpu(), vc.cpu(), _cu([1] * B), seqlens_k=lens,
                      block_table=bt.tolist(), block_size=bs, scale=hd ** -0.5)
    _check(out.view(B, H, hd), ref, f"decode-{H}-{Hkv}-{hd}")


@pytest.mark.parametrize("lq", [[1, 4, 16, 3], [40, 7, 120, 300]])
def test_chunked_append_paged_matches_oracle(lq):
    """flash_attn_varlen_func with a block table: new chunks attend to their
    cached prefix plus themselves, bottom-right causal (paged_llm.py:91-140)."""
    from nanovllm_dots_amd.paged_attention import flash_attn_varlen_func
    H, Hkv, hd, bs = 12, 2, 128, 256
    cached = [0, 300, 511, 1024]
    lk = [c + n for c, n in zip(cached, lq)]
    print(f"append lq={lq} lk={lk}", flush=True)
    kc, vc, bt = _paged(lk, Hkv, hd, bs, seed=sum(lq))
    q = _bf(torch.randn(sum(lq), H, hd, generator=torch.Generator().manual_seed(2)))
    out = flash_attn_varlen_func(q, kc, vc, cu_seqlens_q=_cu(lq).cuda(), cu_seqlens_k=_cu(lk).cuda(),
                                 max_seqlen_q=max(lq), max_seqlen_k=max(lk),
                                 softmax_scale=hd ** -0.5, causal=True, block_table=bt.cuda())
    ref = P.attention(q.cpu(), kc.cpu(), vc.cpu(), _cu(lq), seqlens_k=lk, block_table=bt.tolist(), block_size=bs,
                      scale=hd ** -0.5)
    _check(out, ref, f"append-{lq}")


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_contiguous_matches_oracle(causal):
    """flash_attn_varlen_func without a block table (fresh prefill)."""
    from nanovllm_dots_amd.paged_attention import flash_attn_varlen_func
    H, Hkv, hd = 12, 2, 128
    lens = [5, 64, 1, 333, 97]
    print(f"prefill causal={causal} lens={lens}", flush=True)
    g = torch.Generator().manual_seed(3)
    tot = sum(lens)
    q = _bf(torch.randn(tot, H, hd, generator=g))
    k = _bf(torch.randn(tot, Hkv, hd, generator=g))
    v = _bf(torch.randn(tot, Hkv, hd, generator=g))
    cu = _cu(lens)
    out = flash_attn_varlen_func(q, k, v, cu.cuda(), cu.cuda(), max(lens), max(lens), softmax_scale=0.1,
                                 causal=causal)
    ref = P.attention(q.cpu(), k.cpu(), v.cpu(), cu, cu_k=cu, scale=0.1, causal=causal)
    _check(out, ref, f"prefill-{causal}")


def _ws_bytes(B, H, Hkv, hd, max_q, max_k, total_q):
    import ctypes as C

    from nanovllm_dots_amd import _lib
    a = _lib.DfhPagedAttnArgs(batch=B, num_heads=H, num_kv_heads=Hkv, head_dim=hd, max_seqlen_q=max_q,
                              max_seqlen_k=max_k, total_q=total_q)
    return _lib.lib().dfh_paged_attention_workspace(C.byref(a))


def test_mixed_prefill_workspace_sized_by_rows():
    """One long prompt and many short ones in one prefill (the scheduler's
    16384-token budget allows 4096 + 511 x 24): the workspace follows the
    batch's query rows, not batch x the longest prompt, and the output matches."""
    from nanovllm_dots_amd.paged_attention import flash_attn_varlen_func
    H, Hkv, hd = 12, 2, 128
    # the scheduler's worst case (sizes only, no launch): 3,580 row tiles x 2 KV heads fill the GPU, so
    # one chunk per tile and only the item list; a 32 K-token prompt alike
    sized = _ws_bytes(512, H, Hkv, hd, 4096, 4096, 4096 + 511 * 24)
    long_prompt = _ws_bytes(1, H, Hkv, hd, 32768, 32768, 32768)
    # decode of 512 sequences at 4096 keys keeps the split (partial sums of 16.6 KB per row tile and chunk)
    decode = _ws_bytes(512, H, Hkv, hd, 1, 4096, 512)
    print(f"workspace: 4096 + 511 x 24 prefill {sized / 2**10:.1f} KiB, 32 K prompt {long_prompt / 2**10:.1f} KiB, "
          f"512-sequence decode {decode / 2**20:.1f} MiB", flush=True)
    assert sized < 2**20 and long_prompt < 2**20 and decode < 2**28
    # a smaller instance of the same shape, run against the oracle
    lens = [1500] + [24] * 60
    print(f"mixed prefill lens=[1500] + [24] x 60", flush=True)
    g = torch.Generator().manual_seed(6)
    tot = sum(lens)
    q = _bf(torch.randn(tot, H, hd, generator=g))
    k = _bf(torch.randn(tot, Hkv, hd, generator=g))
    v = _bf(torch.randn(tot, Hkv, hd, generator=g))
    cu = _cu(lens)
    out = flash_attn_varlen_func(q, k, v, cu.cuda(), cu.cuda(), max(lens), max(lens), causal=True)
    ref = P.attention(q.cpu(), k.cpu(), v.cpu(), cu, cu_k=cu, causal=True)
    _check(out, ref, "mixed-prefill")


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_one_chunk_direct_output(causal):
    """Row tiles alone fill the GPU: one chunk per tile, the attention kernel
    writes the normalised rows itself (no partial sums, no combine), and the
    workspace holds only the item list."""
    from nanovllm_dots_amd.paged_attention import flash_attn_varlen_func
    H, Hkv, hd = 32, 32, 64
    lens = [1500, 1400, 1600, 3]
    tot = sum(lens)
    assert _ws_bytes(len(lens), H, Hkv, hd, max(lens), max(lens), tot) < 4096
    print(f"direct prefill causal={causal} lens={lens}", flush=True)
    g = torch.Generator().manual_seed(7)
    q = _bf(torch.randn(tot, H, hd, generator=g))
    k = _bf(torch.randn(tot, Hkv, hd, generator=g))
    v = _bf(torch.randn(tot, Hkv, hd, generator=g))
    cu = _cu(lens)
    out = flash_attn_varlen_func(q, k, v, cu.cuda(), cu.cuda(), max(lens), max(lens), causal=causal)
    ref = P.attention(q.cpu(), k.cpu(), v.cpu(), cu, cu_k=cu, causal=causal)
    _check(out, ref, f"direct-prefill-{causal}")


def test_decode_long_context_and_contiguous_cache():
    """Many chunks per row (8197 keys), and flash_attn_with_kvcache on a
    contiguous [B, S, H_kv, hd] cache (no block table)."""
    from nanovllm_dots_amd.paged_attention import flash_attn_with_kvcache
    H, Hkv, hd, S = 12, 2, 128, 8197
    lens = [8197, 4100, 17]
    print(f"long decode lens={lens}", flush=True)
    g = torch.Generator().manual_seed(4)
    kc = _bf(torch.randn(3, S, Hkv, hd, generator=g))
    vc = _bf(torch.randn(3, S, Hkv, hd, generator=g))
    q = _bf(torch.randn(3, 2, H, hd, generator=g))
    out = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor(lens, dtype=torch.int32).cuda(),
                                  causal=True)
    cu_k = torch.tensor([0, S, 2 * S, 3 * S])
    ref = P.attention(q.reshape(6, H, hd).cpu(), kc.reshape(3 * S, Hkv, hd).cpu(),
                      vc.reshape(3 * S, Hkv, hd).cpu(), _cu([2, 2, 2]), cu_k=cu_k, seqlens_k=lens)
    _check(out.reshape(6, H, hd), ref, "long-decode")


def test_store_kvcache_bit_exact_and_skips():
    from nanovllm_dots_amd.paged_attention import store_kvcache
    N, Hkv, hd, bs, pages = 37, 2, 128, 256, 3
    g = torch.Generator().manual_seed(5)
    key = _bf(torch.randn(N, Hkv, hd, generator=g))
    val = _bf(torch.randn(N, Hkv, hd, generator=g))
    slots = torch.randperm(pages * bs, generator=g)[:N].to(torch.int32)
    slots[::5] = -1
    kc = torch.zeros(pages, bs, Hkv, hd, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    print(f"store_kvcache N={N}", flush=True)
    store_kvcache(key, val, kc, vc, slots.cuda())
    rk, rv = torch.zeros_like(kc).cpu(), torch.zeros_like(vc).cpu()
    P.store_kvcache(key.cpu(), val.cpu(), rk, rv, slots)
    assert torch.equal(kc.cpu(), rk) and torch.equal(vc.cpu(), rv)
    # strided key / value views (a slice of a fused qkv output) store the same rows
    qkv = _bf(torch.randn(N, 3, Hkv, hd, generator=g))
    kc.zero_(), vc.zero_()
    store_kvcache(qkv[:, 1], qkv[:, 2], kc, vc, slots.cuda())
    rk.zero_(), rv.zero_()
    P.store_kvcache(qkv[:, 1].cpu(), qkv[:, 2].cpu(), rk, rv, slots)
    assert torch.equal(kc.cpu(), rk) and torch.equal(vc.cpu(), rv)


def test_rejected_inputs():
    import ctypes as C

    from nanovllm_dots_amd import _lib
    from nanovllm_dots_amd.paged_attention import flash_attn_varlen_func
    H, Hkv, hd = 4, 2, 96
    q = _bf(torch.randn(3, H, hd))
    k = _bf(torch.randn(3, Hkv, hd))
    cu = _cu([3]).cuda()
    with pytest.raises(RuntimeError, match="head_dim"):
        flash_attn_varlen_func(q, k, k, cu, cu, 3, 3, causal=True)
    with pytest.raises(NotImplementedError):
        flash_attn_varlen_func(q, k, k, cu, cu, 3, 3, causal=True, window_size=(8, 0))
    # pages that are not a multiple of 256 tokens, and a short workspace
    lib = _lib.lib()
    hd = 64
    q = _bf(torch.randn(1, 2, hd))
    kc = _bf(torch.randn(2, 128, 1, hd))
    bt = torch.tensor([[0, 1]], dtype=torch.int32).cuda()
    lens = torch.tensor([100], dtype=torch.int32).cuda()
    out = torch.empty_like(q)
    ws = torch.empty(1 << 16, device="cuda")
    a = _lib.DfhPagedAttnArgs(batch=1, num_heads=2, num_kv_heads=1, head_dim=hd, max_seqlen_q=1, max_seqlen_k=256,
                              q=_lib.ptr(q), q_stride=2 * hd, cu_seqlens_q=_lib.ptr(_cu([1]).cuda()), k=_lib.ptr(kc),
                              v=_lib.ptr(kc), kv_stride=hd, cu_seqlens_k=None, seqlens_k=_lib.ptr(lens),
                              block_table=_lib.ptr(bt), block_table_stride=2, block_size=128, out=_lib.ptr(out),
                              out_stride=2 * hd, softmax_scale=0.125, causal=1, workspace=_lib.ptr(ws),
                              workspace_bytes=ws.numel() * 4)
    assert lib.dfh_paged_attention(C.byref(a), _lib.stream_ptr()) != 0
    assert b"block_size" in lib.dfh_last_error()
    a.block_size = 256
    a.workspace_bytes = 16
    assert lib.dfh_paged_attention(C.byref(a), _lib.stream_ptr()) != 0
    assert b"workspace" in lib.dfh_last_error()
