"""ctypes binding of libdotsfm.so (include/dots_fm.h).

The library is required: loading fails loudly when it is missing or when no
GPU is visible. There is no CPU or torch fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdotsfm.so")

vp = C.c_void_p


class DfhConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("heads", C.c_int), ("head_dim", C.c_int), ("ffn", C.c_int),
        ("n_blocks", C.c_int), ("latent_dim", C.c_int), ("patch", C.c_int), ("freq_dim", C.c_int),
        ("qkv_bias", C.c_int), ("qk_norm", C.c_int), ("rotary", C.c_int), ("meanflow", C.c_int),
        ("ln_eps", C.c_float),
        ("rope_inv_freq", C.POINTER(C.c_float)), ("temb_freqs", C.POINTER(C.c_float)),
    ]


class DfhBlockWeights(C.Structure):
    _fields_ = [(n, vp) for n in (
        "q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "q_norm_w", "q_norm_b", "k_norm_w", "k_norm_b",
        "o_w", "o_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b", "ada_w", "ada_b")]


class DfhWeights(C.Structure):
    _fields_ = [(n, vp) for n in (
        "input_w", "input_b", "t_w0", "t_b0", "t_w2", "t_b2", "d_w0", "d_b0", "d_w2", "d_b2",
        "final_ada_w", "final_ada_b", "final_w", "final_b", "coord_w", "coord_b")] + [
        ("blocks", C.POINTER(DfhBlockWeights))]


class DfhSolveArgs(C.Structure):
    _fields_ = [
        ("n", C.c_int), ("total_len", C.c_int), ("num_steps", C.c_int),
        ("input_sequence", vp), ("pos_ids", vp), ("g_cond", vp), ("noise", vp), ("out", vp),
        ("t_grid", C.POINTER(C.c_float)), ("dt_grid", C.POINTER(C.c_float)),
    ]


class DfhVarlenSolveArgs(C.Structure):
    _fields_ = [
        ("n", C.c_int), ("max_hist", C.c_int), ("num_steps", C.c_int),
        ("hist_rows", vp), ("hist_len", vp), ("row_stride", C.c_long),
        ("g_cond", vp), ("noise", vp), ("out", vp),
        ("t_grid", C.POINTER(C.c_float)), ("dt_grid", C.POINTER(C.c_float)),
    ]


class DfhPagedAttnArgs(C.Structure):
    _fields_ = [
        ("batch", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int), ("head_dim", C.c_int),
        ("max_seqlen_q", C.c_int), ("max_seqlen_k", C.c_int),
        ("q", vp), ("q_stride", C.c_long), ("cu_seqlens_q", vp),
        ("k", vp), ("v", vp), ("kv_stride", C.c_long),
        ("cu_seqlens_k", vp), ("seqlens_k", vp), ("block_table", vp),
        ("block_table_stride", C.c_int), ("block_size", C.c_int),
        ("out", vp), ("out_stride", C.c_long), ("softmax_scale", C.c_float), ("causal", C.c_int),
        ("workspace", vp), ("workspace_bytes", C.c_long), ("total_q", C.c_long),
    ]


class DfhPatchEncConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("latent_dim", "patch", "hidden", "heads", "ffn", "n_layers", "out_dim",
                                        "max_batch", "capacity")] + [("ln_eps", C.c_float)]


class DfhPatchEncLayerWeights(C.Structure):
    _fields_ = [(n, vp) for n in ("attn_norm_w", "attn_norm_b", "q_w", "k_w", "v_w", "o_w", "o_b", "ffn_norm_w",
                                  "ffn_norm_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class DfhPatchEncWeights(C.Structure):
    _fields_ = [(n, vp) for n in ("ds_w", "ds_b", "in_w", "in_b", "out_w", "out_b")] + [
        ("layers", C.POINTER(DfhPatchEncLayerWeights))]


class DfhInt8Linear(C.Structure):
    _fields_ = [("w", vp), ("scale", vp)]


class DfhInt8Weights(C.Structure):
    _fields_ = [("input", DfhInt8Linear), ("t_mlp2", DfhInt8Linear), ("d_mlp2", DfhInt8Linear),
                ("ada", DfhInt8Linear)] + [(n, C.POINTER(DfhInt8Linear)) for n in ("qkv", "o", "fc1", "fc2")]


class DfhForwardArgs(C.Structure):
    _fields_ = [
        ("n", C.c_int), ("total_len", C.c_int), ("x", vp), ("timesteps", vp), ("duration", vp),
        ("pos_ids", vp), ("g_cond", vp), ("out", vp),
    ]


# exported symbol -> (restype, argtypes); every symbol here is declared in include/dots_fm.h
SIGNATURES = {
    "dfh_last_error": (C.c_char_p, []),
    "dfh_create": (C.c_int, [C.POINTER(DfhConfig), C.POINTER(vp)]),
    "dfh_destroy": (C.c_int, [vp]),
    "dfh_set_weights": (C.c_int, [vp, C.POINTER(DfhWeights), vp]),
    "dfh_reserve": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, vp]),
    "dfh_meanflow_solve": (C.c_int, [vp, C.POINTER(DfhSolveArgs), vp]),
    "dfh_meanflow_solve_varlen": (C.c_int, [vp, C.POINTER(DfhVarlenSolveArgs), vp]),
    "dfh_dit_forward": (C.c_int, [vp, C.POINTER(DfhForwardArgs), vp]),
    "dfh_input_status": (C.c_int, [vp, C.POINTER(C.c_int), vp]),
    "dfh_profile_enable": (C.c_int, [vp, C.c_int]),
    "dfh_set_ksplit": (C.c_int, [vp, C.c_int]),
    "dfh_set_ln_quant": (C.c_int, [vp, C.c_int]),
    "dfh_profile_classes": (C.c_int, [vp, C.c_uint, C.c_int]),
    "dfh_set_latent_tail": (C.c_int, [vp, C.c_int]),
    "dfh_set_int8": (C.c_int, [vp, C.c_int, vp, vp]),
    "dfh_profile_read": (C.c_int, [vp, C.POINTER(C.c_double), C.POINTER(C.c_long), C.c_int]),
    "dfh_gemm_bf16": (C.c_int, [vp, C.c_long, vp, C.c_long, vp, C.c_long, vp, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, vp]),
    "dfh_gemm_bf16_ws": (C.c_int, [vp, C.c_long, vp, C.c_long, vp, C.c_long, vp, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, vp, C.c_long, vp]),
    "dfh_quant_act_i8": (C.c_int, [vp, C.c_long, vp, C.c_long, vp, C.c_int, C.c_int, vp]),
    "dfh_quant_weight_i8": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, vp]),
    "dfh_gemm_w8a8": (C.c_int, [vp, C.c_long, vp, C.c_long, vp, C.c_long, vp, vp, vp, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, vp]),
    "dfh_gemm_w8a8_ws": (C.c_int, [vp, C.c_long, vp, C.c_long, vp, C.c_long, vp, vp, vp, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, vp, C.c_long, vp]),
    "dfh_store_kvcache": (C.c_int, [vp, C.c_long, vp, C.c_long, vp, vp, vp, C.c_int, C.c_int, vp]),
    "dfh_paged_attention_workspace": (C.c_long, [C.POINTER(DfhPagedAttnArgs)]),
    "dfh_paged_attention": (C.c_int, [C.POINTER(DfhPagedAttnArgs), vp]),
    "dfh_paged_attention_noalloc": (C.c_int, [C.POINTER(DfhPagedAttnArgs), vp]),
    "dfh_kvcache_create": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, C.POINTER(vp)]),
    "dfh_kvcache_destroy": (C.c_int, [vp]),
    "dfh_kvcache_reset": (C.c_int, [vp, vp]),
    "dfh_kvcache_lengths": (C.c_int, [vp, C.POINTER(C.c_int)]),
    "dfh_kvcache_extend": (C.c_int, [vp, vp, C.c_int, C.POINTER(C.c_int), vp, C.POINTER(C.c_float),
                                     C.POINTER(C.c_float), vp]),
    "dfh_kvcache_solve": (C.c_int, [vp, vp, vp, vp, vp, C.POINTER(C.c_float), C.POINTER(C.c_float), vp]),
    "dfh_patchenc_create": (C.c_int, [C.POINTER(DfhPatchEncConfig), C.POINTER(DfhPatchEncWeights), C.POINTER(vp)]),
    "dfh_patchenc_destroy": (C.c_int, [vp]),
    "dfh_patchenc_reset_rows": (C.c_int, [vp, vp, C.c_int, vp]),
    "dfh_patchenc_decode": (C.c_int, [vp, vp, C.c_long, vp, C.c_int, vp, vp]),
    "dfh_patchenc_lengths": (C.c_int, [vp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
}

_lib = None


def load_library(path: str = LIB_PATH):
    """dlopen the library and bind every declared symbol (no GPU needed)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"libdotsfm.so not found at {path}; build it with `python -m nanovllm_dots_amd.build`")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def lib():
    """The library, for a GPU call: raises when no GPU is visible."""
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("nanovllm_dots_amd needs a ROCm GPU (gfx950); none is visible")
    return load_library()


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = load_library().dfh_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}" if what else msg)


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return vp(s.cuda_stream)


def ptr(t) -> vp:
    return vp(t.data_ptr()) if t is not None else vp(None)
