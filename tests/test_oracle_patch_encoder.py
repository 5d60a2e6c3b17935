"""The patch encoder oracle against the fixture the reference's own
native/patch_encoder.py wrote (tests/golden/patch_encoder.npz), and the batched
cache-row bookkeeping of FlashPatchEncoder against per-request decodes. CPU."""
from __future__ import annotations

import ast

import numpy as np
import torch

from conftest import load_golden
from oracle import patch_encoder_ref as PE


def _fixture():
    g = load_golden("patch_encoder.npz")
    cfg = PE.PatchEncConfig(**ast.literal_eval(str(g["cfg"])))
    return g, cfg, PE.random_pe_weights(cfg, int(g["seed"]))


def test_decode_matches_reference_fixture():
    g, cfg, W = _fixture()
    for i, n in enumerate(g["steps"]):
        st = PE.init_state(cfg, 16 * cfg.ods)
        for t in range(int(n)):
            e = PE.decode_patch(W, cfg, torch.from_numpy(g["patches"][i, t]), st)
            ref = torch.from_numpy(g["emb"][i, t])
            err = (e - ref).abs().max().item()
            assert err <= 2e-5 * ref.abs().max().item(), (i, t, err)
        assert st.seq_len == int(n) * cfg.ods
        assert torch.equal(st.conv_tail[:, 0], torch.from_numpy(g["tails"][i]))


def test_batched_rows_equal_per_request_decodes():
    """Rows in a shuffled order, requests at different history lengths in one
    call (the continuous-batching case of flash_patch_encoder.py:103-139)."""
    g, cfg, W = _fixture()
    rs = np.random.RandomState(3)
    cache = PE.PatchEncoderCacheRef(W, cfg, max_batch=4, cap=32 * cfg.ods)
    solo = [PE.init_state(cfg, 32 * cfg.ods) for _ in range(4)]
    plan = [[2, 0], [0, 3, 1], [3], [1, 2, 0, 3]]
    for rows in plan:
        patches = torch.from_numpy(rs.standard_normal((len(rows), cfg.patch, cfg.latent_dim)).astype(np.float32))
        got = cache.decode_patch(patches, rows)
        for i, r in enumerate(rows):
            ref = PE.decode_patch(W, cfg, patches[i], solo[r])
            assert torch.allclose(got[i, 0], ref, rtol=0, atol=1e-6)
    assert [cache.seqlen(r) for r in range(4)] == [s.seq_len for s in solo]
    cache.reset_rows([1])
    assert cache.seqlen(1) == 0 and torch.equal(cache.rows[1].conv_tail, torch.zeros(cfg.latent_dim, 1))


def test_history_changes_the_embedding():
    """The cache is read: the same patch after different histories embeds
    differently, and the conv tail carries the previous patch's last frame."""
    _, cfg, W = _fixture()
    rs = np.random.RandomState(4)
    p = [torch.from_numpy(rs.standard_normal((cfg.patch, cfg.latent_dim)).astype(np.float32)) for _ in range(3)]
    a, b = PE.init_state(cfg, 8 * cfg.ods), PE.init_state(cfg, 8 * cfg.ods)
    PE.decode_patch(W, cfg, p[0], a)
    PE.decode_patch(W, cfg, p[1], b)
    assert torch.equal(a.conv_tail[:, 0], p[0][-1])
    ea, eb = PE.decode_patch(W, cfg, p[2], a), PE.decode_patch(W, cfg, p[2], b)
    assert (ea - eb).abs().max().item() > 1e-3


def test_wrapper_reads_dims_off_the_module():
    """HipPatchEncoder takes the reference module as FlashPatchEncoder does
    (flash_patch_encoder.py:43-62) and reads the shapes off it."""
    from types import SimpleNamespace as NS

    from nanovllm_dots_amd.patch_encoder import _dims_of
    layer = NS(attn=NS(num_heads=16), ffn=NS(fc1=NS(out_features=4096)), attn_norm=NS(eps=1e-5))
    pe = NS(ds_proj=NS(in_channels=64), patch_size=16, encoder=NS(hidden_size=1024, layers=[layer] * 6),
            out_proj=NS(out_features=1536))
    assert _dims_of(pe) == dict(latent_dim=64, patch=16, hidden=1024, heads=16, ffn=4096, n_layers=6,
                                out_dim=1536, ln_eps=1e-5)
