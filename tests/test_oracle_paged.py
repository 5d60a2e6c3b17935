"""Pins the paged-attention oracle (CPU) against a library routine, the
chunked-append invariant and closed forms."""
from __future__ import annotations

import torch

from oracle import paged_attn_ref as P


def _sdpa(q, k, v, cu_q, cu_k, causal):
    """torch SDPA in float64 with an explicit bottom-right mask, KV heads repeated."""
    H, Hkv = q.shape[1], k.shape[1]
    out = torch.zeros(q.shape, dtype=torch.float64)
    for i in range(len(cu_q) - 1):
        q0, q1, k0, k1 = int(cu_q[i]), int(cu_q[i + 1]), int(cu_k[i]), int(cu_k[i + 1])
        Lq, Lk = q1 - q0, k1 - k0
        Q = q[q0:q1].double().transpose(0, 1)
        K = k[k0:k1].double().repeat_interleave(H // Hkv, dim=1).transpose(0, 1)
        V = v[k0:k1].double().repeat_interleave(H // Hkv, dim=1).transpose(0, 1)
        mask = torch.ones(Lq, Lk, dtype=torch.bool)
        if causal:
            mask = torch.ones(Lq, Lk, dtype=torch.bool).tril(diagonal=Lk - Lq)
        o = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask)
        out[q0:q1] = o.transpose(0, 1)
    return out


def _rand(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def test_matches_sdpa_gqa_bottom_right():
    H, Hkv, hd = 6, 2, 16
    lq, lk = [1, 3, 5, 4], [7, 3, 9, 12]
    cu_q = torch.tensor([0] + list(torch.tensor(lq).cumsum(0)))
    cu_k = torch.tensor([0] + list(torch.tensor(lk).cumsum(0)))
    q = _rand(int(cu_q[-1]), H, hd, seed=1)
    k = _rand(int(cu_k[-1]), Hkv, hd, seed=2)
    v = _rand(int(cu_k[-1]), Hkv, hd, seed=3)
    for causal in (True, False):
        got = P.attention(q, k, v, cu_q, cu_k=cu_k, causal=causal)
        ref = _sdpa(q, k, v, cu_q, cu_k, causal)
        assert torch.allclose(got, ref, atol=1e-12), causal


def test_chunked_append_equals_full_prefill():
    """Appending a sequence in chunks (bottom-right causal) gives the rows of one
    full causal prefill: a top-left alignment would fail this."""
    H, Hkv, hd, L = 4, 1, 8, 23
    q = _rand(L, H, hd, seed=4)
    k = _rand(L, Hkv, hd, seed=5)
    v = _rand(L, Hkv, hd, seed=6)
    full = P.attention(q, k, v, torch.tensor([0, L]), cu_k=torch.tensor([0, L]))
    start = 0
    for chunk in (5, 1, 9, 8):
        end = start + chunk
        part = P.attention(q[start:end], k[:end], v[:end], torch.tensor([0, chunk]), cu_k=torch.tensor([0, end]))
        assert torch.allclose(part, full[start:end], atol=1e-12), (start, end)
        start = end


def test_paged_equals_contiguous_under_page_permutation():
    H, Hkv, hd, bs = 4, 2, 8, 4
    lk = [9, 4, 1]
    lq = [2, 4, 1]
    total = sum(lk)
    k = _rand(total, Hkv, hd, seed=7)
    v = _rand(total, Hkv, hd, seed=8)
    cu_k = torch.tensor([0] + list(torch.tensor(lk).cumsum(0)))
    cu_q = torch.tensor([0] + list(torch.tensor(lq).cumsum(0)))
    q = _rand(sum(lq), H, hd, seed=9)
    # scatter every sequence's keys into shuffled physical pages
    n_pages = sum((L + bs - 1) // bs for L in lk) + 2
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(10)).tolist()
    kc = torch.full((n_pages, bs, Hkv, hd), float("nan"), dtype=torch.float64)
    vc = kc.clone()
    tables, nxt = [], 0
    for i, L in enumerate(lk):
        pages = perm[nxt:nxt + (L + bs - 1) // bs]
        nxt += len(pages)
        tables.append(pages + [-1] * (4 - len(pages)))
        for t in range(L):
            kc[pages[t // bs], t % bs] = k[int(cu_k[i]) + t]
            vc[pages[t // bs], t % bs] = v[int(cu_k[i]) + t]
    paged = P.attention(q, kc, vc, cu_q, seqlens_k=torch.tensor(lk), block_table=tables, block_size=bs)
    cont = P.attention(q, k, v, cu_q, cu_k=cu_k)
    assert torch.allclose(paged, cont, atol=1e-12)


def test_closed_forms():
    hd = 8
    v = _rand(5, 1, hd, seed=11)
    # one visible key: the output is that key's V row
    q = _rand(1, 1, hd, seed=12)
    k = _rand(5, 1, hd, seed=13)
    out = P.attention(q, k[:1], v[:1], torch.tensor([0, 1]), cu_k=torch.tensor([0, 1]))
    assert torch.allclose(out[0, 0], v[0, 0], atol=1e-14)
    # equal keys: the output is the mean of the visible V rows
    keq = k[:1].repeat(5, 1, 1)
    out = P.attention(q, keq, v, torch.tensor([0, 1]), cu_k=torch.tensor([0, 5]))
    assert torch.allclose(out[0, 0], v[:, 0].mean(0), atol=1e-12)
    # Lk < Lq under the causal rule: rows that see no key are 0
    out = P.attention(_rand(3, 1, hd, seed=14), k[:1], v[:1], torch.tensor([0, 3]), cu_k=torch.tensor([0, 1]))
    assert torch.equal(out[:2], torch.zeros(2, 1, hd, dtype=torch.float64))


def test_store_kvcache_slots():
    key = _rand(4, 2, 8, seed=15)
    val = _rand(4, 2, 8, seed=16)
    kc = torch.zeros(3, 4, 2, 8, dtype=torch.float64)
    vc = torch.zeros_like(kc)
    P.store_kvcache(key, val, kc, vc, torch.tensor([5, -1, 0, 11]))
    flat = kc.view(-1, 16)
    assert torch.equal(flat[5], key[0].reshape(-1))
    assert torch.equal(flat[0], key[2].reshape(-1))
    assert torch.equal(flat[11], key[3].reshape(-1))
    assert int((flat.abs().sum(1) > 0).sum()) == 3
    assert torch.equal(vc.view(-1, 16)[11], val[3].reshape(-1))
