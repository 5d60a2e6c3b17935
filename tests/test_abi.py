"""The C ABI library loads on the CPU and exports every entry point that
include/dots_fm.h declares (no compute call is made here)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dots_fm.h")
LIB = os.path.join(ROOT, "nanovllm_dots_amd", "libdotsfm.so")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dfh_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libdotsfm.so is not built (python -m nanovllm_dots_amd.build)")
    return ctypes.CDLL(LIB)


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("dfh_create", "dfh_meanflow_solve", "dfh_dit_forward", "dfh_gemm_bf16", "dfh_last_error"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_covers_header():
    from nanovllm_dots_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_exports_are_c_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (dfh_[a-z0-9_]+)\b", out))
    assert set(declared_symbols()) <= exported


def test_library_carries_gfx950_code_object():
    """The .hip_fatbin section of our own build names the gfx950 target."""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "fatbin")
        r = subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", LIB, out],
                           capture_output=True, text=True)
        if r.returncode != 0:
            pytest.skip("objcopy unavailable")
        data = open(out, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_paged_wrappers_take_flash_attn_positional_order():
    """flash-attn 2.8.3's parameter lists (positional order and names), so a
    positional call from layers/attention.py binds the same arguments."""
    import inspect

    from nanovllm_dots_amd import paged_attention as PA
    varlen = ["q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k", "dropout_p",
              "softmax_scale", "causal", "window_size", "softcap", "alibi_slopes", "deterministic",
              "return_attn_probs", "block_table"]
    kvcache = ["q", "k_cache", "v_cache", "k", "v", "rotary_cos", "rotary_sin", "cache_seqlens",
               "cache_batch_idx", "cache_leftpad", "block_table", "softmax_scale", "causal", "window_size",
               "softcap", "rotary_interleaved", "alibi_slopes", "num_splits", "return_softmax_lse"]
    assert list(inspect.signature(PA.flash_attn_varlen_func).parameters) == varlen
    assert list(inspect.signature(PA.flash_attn_with_kvcache).parameters) == kvcache
