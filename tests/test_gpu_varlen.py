"""Varlen solve (``dfh_meanflow_solve_varlen``): requests handed over as the
engine holds them (per-request history tensors and lengths), in place of the
padded batch that DotsBatchEngine._pack_fm_inputs builds (engine.py:635-688).
GPU only.

Bar: bit-identical latents to ``dfh_meanflow_solve`` on the padded batch of the
same requests (the packed rows, row tables and kernels are the same), and the
oracle's tolerance (per-row cosine >= 0.9999, max |diff| <= 0.02 * max |ref|)
against ``meanflow_solve_varlen`` of the oracle."""
from __future__ import annotations

import ctypes as C

import pytest
import torch

from oracle import dit_ref as R
from test_gpu_parity import FULL, VARIANTS, _assert_latents, _assert_vs_fp32, _cuda_bf16, _head, _inputs

pytestmark = pytest.mark.gpu


def _engine_states(hist, extra_rows, seed):
    """fm_sequence-like tensors: [1, capacity, H] bf16 with the history in the
    first c_i rows and non-zero junk after it (the solve must not read it)."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for h in hist:
        cap = h.shape[0] + extra_rows
        t = torch.randn(1, cap, h.shape[1], generator=g) * 7.0
        t[0, :h.shape[0]] = h
        out.append(_cuda_bf16(t))
    return out


@pytest.mark.parametrize("name", ["rope", "qknorm_bias"])
def test_varlen_equals_padded_bit_exact(name):
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS[name]
    head, Wb = _head(cfg, seed=12)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 6, 1, 170, seed=13)
    print(f"varlen {name} lens={lens}", flush=True)
    padded = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(g),
                noise=_cuda_bf16(noise))
    seqs = _engine_states(hist, extra_rows=9, seed=14)
    got = mf.solve_varlen(sequences=seqs, lengths=lens, g_cond=_cuda_bf16(g), noise=_cuda_bf16(noise))
    assert torch.equal(got, padded)
    ref = R.meanflow_solve_varlen(Wb, cfg, hist, g, noise, 4, "bf16")
    _assert_latents(got, ref, cfg.latent_dim, f"varlen-{name}")
    _assert_vs_fp32(got, Wb, cfg, hist, g, noise, f"varlen-{name}")


def test_varlen_mixed_strides_and_views():
    """2-D views with different row strides fall back to packed copies; 3-D
    [1, L, H] tensors are accepted; the result does not change."""
    from nanovllm_dots_amd import HipMeanflow
    cfg = VARIANTS["rope"]
    head, _ = _head(cfg, seed=15)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 3, 2, 60, seed=16)
    padded = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=None,
                noise=_cuda_bf16(noise))
    wide = [_cuda_bf16(torch.cat([h, torch.zeros(h.shape[0], 8 * (i + 1))], dim=1))[:, :cfg.hidden]
            for i, h in enumerate(hist)]
    assert len({w.stride(0) for w in wide}) == 3
    got = mf.solve_varlen(sequences=wide, lengths=lens, g_cond=None, noise=_cuda_bf16(noise))
    assert torch.equal(got, padded)
    got3 = mf.solve_varlen(sequences=[_cuda_bf16(h)[None] for h in hist], lengths=lens, noise=_cuda_bf16(noise))
    assert torch.equal(got3, padded)


def test_varlen_bad_inputs_raise():
    from nanovllm_dots_amd import HipMeanflow, _lib
    cfg = VARIANTS["rope"]
    head, _ = _head(cfg, seed=17)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    lens, hist, noise, *_ = _inputs(cfg, 2, 5, 9, seed=18)
    seqs = [_cuda_bf16(h) for h in hist]
    with pytest.raises(RuntimeError, match="outside"):
        mf.solve_varlen(sequences=seqs, lengths=[lens[0], lens[1] + 1], noise=_cuda_bf16(noise))
    with pytest.raises(RuntimeError, match="nfe"):
        mf.solve_varlen(sequences=seqs, lengths=lens, num_steps=2, noise=_cuda_bf16(noise))
    # a device-side length outside [1, max_hist] is flagged by dfh_input_status
    lib = head.lib
    ptrs = torch.tensor([s.data_ptr() for s in seqs], dtype=torch.int64).cuda()
    bad = torch.tensor([lens[0], 0], dtype=torch.int32).cuda()
    out = torch.empty((2, cfg.patch, cfg.latent_dim), device="cuda", dtype=torch.bfloat16)
    nz = _cuda_bf16(noise)
    tg = (C.c_float * 4)(0.0, 0.25, 0.5, 0.75)
    dg = (C.c_float * 4)(0.25, 0.25, 0.25, 0.25)
    args = _lib.DfhVarlenSolveArgs(n=2, max_hist=max(lens), num_steps=4, hist_rows=_lib.ptr(ptrs),
                                   hist_len=_lib.ptr(bad), row_stride=cfg.hidden, g_cond=None,
                                   noise=_lib.ptr(nz), out=_lib.ptr(out), t_grid=tg, dt_grid=dg)
    st = _lib.stream_ptr()
    assert lib.dfh_meanflow_solve_varlen(head.handle, C.byref(args), st) == 0
    flags = C.c_int(0)
    assert lib.dfh_input_status(head.handle, C.byref(flags), st) == 0
    assert flags.value & 1
    # host-side rejections: row stride, NULL pointers
    args.row_stride = cfg.hidden - 8
    assert lib.dfh_meanflow_solve_varlen(head.handle, C.byref(args), st) != 0
    assert b"row_stride" in lib.dfh_last_error()
    args.row_stride = cfg.hidden
    args.hist_len = None
    assert lib.dfh_meanflow_solve_varlen(head.handle, C.byref(args), st) != 0
    # the handle stays usable
    good = mf.solve_varlen(sequences=seqs, lengths=lens, noise=nz)
    assert torch.isfinite(good.float()).all()


def test_full_size_varlen_equals_padded():
    """12 blocks, H=1024: 8 requests with contexts U{64..512}, varlen == padded."""
    from nanovllm_dots_amd import HipMeanflow
    cfg = FULL
    head, Wb = _head(cfg, seed=2)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head, strict=True)
    lens, hist, noise, inp, mask, pos, g = _inputs(cfg, 8, 64, 512, seed=19)
    print(f"full varlen lens={lens}", flush=True)
    padded = mf(input_sequence=_cuda_bf16(inp), attn_mask=None, pos_ids=pos.cuda(), g_cond=_cuda_bf16(g),
                noise=_cuda_bf16(noise))
    got = mf.solve_varlen(sequences=_engine_states(hist, extra_rows=3, seed=20), lengths=lens,
                          g_cond=_cuda_bf16(g), noise=_cuda_bf16(noise))
    assert torch.equal(got, padded)
    _assert_vs_fp32(got, Wb, cfg, hist, g, noise, "full varlen", device="cuda")
