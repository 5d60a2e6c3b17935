"""Paged KV cache of the LLM backbone (test infrastructure only).

Restates, on the CPU in float64:

* ``store_kvcache`` (nanovllm_dots/layers/attention.py:10-47): token i's K / V
  rows go to cache row ``slot_mapping[i]``; slot -1 skips the token.
* the attention ``Attention.forward`` gets from flash-attn 2.8.3
  (layers/attention.py:66-95; flash-attn is not vendored): for sequence i,
  queries ``q[cu_q[i]:cu_q[i+1]]`` against Lk_i keys that live either in the
  paged cache (key t at page ``block_table[i][t // block_size]``, offset
  ``t % block_size``) or contiguously at rows ``cu_k[i] + t``. With
  ``causal=True`` the mask is bottom-right aligned (flash-attn's rule when
  seqlen_q != seqlen_k): query j of Lq sees keys ``[0, Lk - Lq + j]``; a row
  that sees no key is 0. Query head h uses KV head ``h // (H / H_kv)``.

Pinned in tests/test_oracle_paged.py against torch's SDPA (float64, explicit
mask, KV heads repeated), the chunked-append == full-prefill invariant that
fixes the bottom-right alignment, paged == contiguous under a page
permutation, and closed forms (one visible key; equal keys).
"""
from __future__ import annotations

import torch


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """In place on ``k_cache`` / ``v_cache`` viewed as [num_slots, D] (attention.py:10-33)."""
    N = key.shape[0]
    kc = k_cache.view(-1, key.shape[1] * key.shape[2])
    vc = v_cache.view(-1, value.shape[1] * value.shape[2])
    for i in range(N):
        s = int(slot_mapping[i])
        if s == -1:
            continue
        kc[s] = key[i].reshape(-1)
        vc[s] = value[i].reshape(-1)


def seq_keys(k, i, Lk, cu_k=None, block_table=None, block_size=None):
    """[Lk, H_kv, hd] keys of sequence i from a paged cache or a contiguous tensor."""
    if block_table is None:
        start = int(cu_k[i])
        return k[start:start + Lk]
    rows = []
    for t in range(Lk):
        page = int(block_table[i][t // block_size])
        rows.append(k[page, t % block_size])
    return torch.stack(rows) if rows else k.new_zeros((0,) + tuple(k.shape[2:]))


def attention(q, k, v, cu_q, *, cu_k=None, seqlens_k=None, block_table=None, block_size=None, scale=None,
              causal=True):
    """float64 [total_q, H, hd] output of the varlen / paged attention."""
    H, hd = q.shape[1], q.shape[2]
    Hkv = k.shape[-2]
    G = H // Hkv
    scale = hd ** -0.5 if scale is None else scale
    out = torch.zeros(q.shape, dtype=torch.float64)
    B = len(cu_q) - 1
    for i in range(B):
        q0, q1 = int(cu_q[i]), int(cu_q[i + 1])
        Lq = q1 - q0
        Lk = int(seqlens_k[i]) if seqlens_k is not None else int(cu_k[i + 1]) - int(cu_k[i])
        K = seq_keys(k, i, Lk, cu_k, block_table, block_size).double()
        V = seq_keys(v, i, Lk, cu_k, block_table, block_size).double()
        Q = q[q0:q1].double()
        t = torch.arange(Lk)
        jj = torch.arange(Lq)
        vis = (t[None, :] <= (Lk - Lq + jj)[:, None]) if causal else torch.ones(Lq, Lk, dtype=torch.bool)
        for h in range(H):
            g = h // G
            s = (Q[:, h] @ K[:, g].T) * scale
            s = s.masked_fill(~vis, float("-inf"))
            m = s.max(dim=1, keepdim=True).values
            m = torch.where(torch.isinf(m), torch.zeros_like(m), m)
            p = torch.exp(s - m)
            den = p.sum(dim=1, keepdim=True)
            o = (p @ V[:, g]) / torch.where(den > 0, den, torch.ones_like(den))
            out[q0:q1, h] = o
    return out
