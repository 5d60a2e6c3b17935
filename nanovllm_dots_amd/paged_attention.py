"""Paged KV cache of the LLM backbone on the HIP kernels.

Drop-ins for what ``nanovllm_dots/layers/attention.py`` imports and calls
(Qwen2.5-1.5B backbone: 12 query heads, 2 KV heads, head_dim 128, 256-token
pages):

* ``store_kvcache(key, value, k_cache, v_cache, slot_mapping)`` — same
  signature and checks as attention.py:36-47 (the Triton kernel :10-33).
* ``flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
  max_seqlen_k, dropout_p=0.0, softmax_scale=None, causal=False, ...,
  block_table=None)`` — the prefill / chunked-append call of attention.py:75-86
  (flash-attn 2.8.3 positional order, argument names and meaning; bottom-right
  causal alignment).
* ``flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None,
  rotary_cos=None, rotary_sin=None, cache_seqlens=None, cache_batch_idx=None,
  cache_leftpad=None, block_table=None, softmax_scale=None, causal=False, ...)``
  — the decode call of attention.py:88-95, in flash-attn 2.8.3's positional
  order (``k``/``v`` appends are not supported: the engine stores K/V with
  ``store_kvcache`` first).

Options that do not change the result are accepted at any value
(``num_splits``, a scheduling hint; ``rotary_interleaved`` without rotary
tables); the others only at their defaults.

Switching the reference to these is an import change in
``layers/attention.py``. bf16 only; head_dim 64 or 128; pages a multiple of
256 tokens (the engine's own constraint, config.py:26).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib

def _check_unsupported(**kw):
    """Options of flash-attn 2.8.3 this path implements only at their defaults."""
    for name, val in kw.items():
        if name == "window_size" and tuple(val) == (-1, -1):
            continue
        if name in ("dropout_p", "softcap") and not val:
            continue
        if name in ("return_attn_probs", "deterministic", "return_softmax_lse") and not val:
            continue
        if val is None:
            continue
        raise NotImplementedError(f"{name}={val!r} is not supported by the HIP paged attention")


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    if N == 0:
        return
    for t in (key, value, k_cache, v_cache):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise RuntimeError("store_kvcache: bf16 GPU tensors expected")
    slots = slot_mapping.to(torch.int32).contiguous()
    lib = _lib.lib()
    _lib.check(lib.dfh_store_kvcache(_lib.ptr(key), key.stride(0), _lib.ptr(value), value.stride(0),
                                     _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(slots), N, D,
                                     _lib.stream_ptr()), "dfh_store_kvcache")


def _run(q, k, v, *, cu_q, max_q, max_k, cu_k=None, seqlens_k=None, block_table=None, block_size=0,
         scale=None, causal=True, out=None):
    total_q, H, hd = q.shape
    Hkv = k.shape[-2]
    if k.shape[-1] != hd or v.shape != k.shape:
        raise RuntimeError(f"k / v shapes {tuple(k.shape)} / {tuple(v.shape)} do not match q {tuple(q.shape)}")
    for t in (q, k, v):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise RuntimeError("paged attention: bf16 GPU tensors expected")
        if t.stride(-1) != 1 or t.stride(-2) != hd:
            raise RuntimeError("paged attention: heads must be contiguous [.., heads, head_dim]")
    kv_stride = k.stride(-3)
    if v.stride(-3) != kv_stride:
        raise RuntimeError("paged attention: k and v must share one token stride")
    if block_table is not None and (k.stride(0) != k.shape[1] * kv_stride or v.stride(0) != v.shape[1] * kv_stride):
        raise RuntimeError("paged attention: pages must be contiguous [num_blocks, block_size, ...]")
    if out is None:
        out = torch.empty((total_q, H, hd), device=q.device, dtype=torch.bfloat16)
    B = cu_q.numel() - 1
    cu_q = cu_q.to(torch.int32).contiguous()
    cu_k = cu_k.to(torch.int32).contiguous() if cu_k is not None else None
    seqlens_k = seqlens_k.to(torch.int32).contiguous() if seqlens_k is not None else None
    bt = block_table.to(torch.int32).contiguous() if block_table is not None else None
    args = _lib.DfhPagedAttnArgs(
        batch=B, num_heads=H, num_kv_heads=Hkv, head_dim=hd, max_seqlen_q=int(max_q), max_seqlen_k=int(max_k),
        q=_lib.ptr(q), q_stride=q.stride(0), cu_seqlens_q=_lib.ptr(cu_q), k=_lib.ptr(k), v=_lib.ptr(v),
        kv_stride=kv_stride, cu_seqlens_k=_lib.ptr(cu_k), seqlens_k=_lib.ptr(seqlens_k), block_table=_lib.ptr(bt),
        block_table_stride=bt.shape[1] if bt is not None else 0, block_size=int(block_size),
        out=_lib.ptr(out), out_stride=out.stride(0), softmax_scale=float(hd ** -0.5 if scale is None else scale),
        causal=int(bool(causal)), workspace=None, workspace_bytes=0, total_q=total_q)
    lib = _lib.lib()
    need = lib.dfh_paged_attention_workspace(C.byref(args))
    ws = torch.empty(max((need + 3) // 4, 64), device=q.device, dtype=torch.float32)
    args.workspace = _lib.ptr(ws)
    args.workspace_bytes = ws.numel() * 4
    _lib.check(lib.dfh_paged_attention(C.byref(args), _lib.stream_ptr()), "dfh_paged_attention")
    return out


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                           softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                           deterministic=False, return_attn_probs=False, block_table=None):
    """out [total_q, H, hd]. With ``block_table``, k / v are the paged caches
    [num_blocks, block_size, H_kv, hd] and ``cu_seqlens_k`` gives key counts."""
    _check_unsupported(dropout_p=dropout_p, window_size=window_size, softcap=softcap, alibi_slopes=alibi_slopes,
                       deterministic=deterministic, return_attn_probs=return_attn_probs)
    bs = k.shape[1] if block_table is not None else 0
    return _run(q, k, v, cu_q=cu_seqlens_q, max_q=max_seqlen_q, max_k=max_seqlen_k, cu_k=cu_seqlens_k,
                block_table=block_table, block_size=bs, scale=softmax_scale, causal=causal)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None, block_table=None,
                            softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                            rotary_interleaved=True, alibi_slopes=None, num_splits=0, return_softmax_lse=False):
    """q [B, Lq, H, hd] -> out [B, Lq, H, hd] over the first ``cache_seqlens[b]``
    keys of each batch row (paged through ``block_table``, else k_cache
    [B, S, H_kv, hd])."""
    if k is not None or v is not None:
        raise NotImplementedError("k / v appends: store them with store_kvcache first")
    _check_unsupported(rotary_cos=rotary_cos, rotary_sin=rotary_sin, cache_batch_idx=cache_batch_idx,
                       cache_leftpad=cache_leftpad, window_size=window_size, softcap=softcap,
                       alibi_slopes=alibi_slopes, return_softmax_lse=return_softmax_lse)
    B, Lq, H, hd = q.shape
    dev = q.device
    if cache_seqlens is None:
        raise RuntimeError("cache_seqlens is required")
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=dev)
    cu_q = torch.arange(0, (B + 1) * Lq, Lq, dtype=torch.int32, device=dev)
    q2 = q.reshape(B * Lq, H, hd)
    if block_table is not None:
        bs = k_cache.shape[1]
        max_k = block_table.shape[1] * bs
        out = _run(q2, k_cache, v_cache, cu_q=cu_q, max_q=Lq, max_k=max_k, seqlens_k=cache_seqlens,
                   block_table=block_table, block_size=bs, scale=softmax_scale, causal=causal)
    else:
        S = k_cache.shape[1]
        cu_k = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=dev)
        kc = k_cache.reshape(B * S, *k_cache.shape[2:])
        vc = v_cache.reshape(B * S, *v_cache.shape[2:])
        out = _run(q2, kc, vc, cu_q=cu_q, max_q=Lq, max_k=S, cu_k=cu_k, seqlens_k=cache_seqlens,
                   scale=softmax_scale, causal=causal)
    return out.view(B, Lq, H, hd)
