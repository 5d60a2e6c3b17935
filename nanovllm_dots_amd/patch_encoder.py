"""The patch encoder's batched per-patch decode on the HIP kernels.

``HipPatchEncoder`` is a drop-in for ``FlashPatchEncoder``
(nanovllm_dots/models/dots/flash_patch_encoder.py:35-139): same constructor
(the patch encoder module, ``max_batch`` cache rows, ``max_seq_len`` tokens per
row, device, dtype), ``reset_rows(rows)`` and ``decode_patch(latent_patches,
rows) -> [n, 1, out_dim]``. Request i of a call uses cache row ``rows[i]`` at
that row's own history length, so requests at different lengths share one call
(continuous batching); each call advances the rows by ``patch // 2`` tokens.
The engine switch is its ``flash_pe`` arm constructing this class instead
(engine.py:205-221).

Everything runs in the library (libdotsfm.so, ``dfh_patchenc_*``): causal
downsample, in_proj, the encoder layers (LayerNorm, fused q|k|v GEMM, K / V
appended to the row's cache, paged attention over the row's keys, o_proj and
MLP GEMMs with fused bias, SiLU and residual epilogues) and out_proj. There is
no CPU or torch fallback.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib

# nn.Module attribute paths of a VAESemanticEncoder (native/patch_encoder.py:144-152)
_LAYER_KEYS = (("attn_norm_w", "attn_norm.weight"), ("attn_norm_b", "attn_norm.bias"),
               ("q_w", "attn.q_proj.weight"), ("k_w", "attn.k_proj.weight"), ("v_w", "attn.v_proj.weight"),
               ("o_w", "attn.o_proj.weight"), ("o_b", "attn.o_proj.bias"),
               ("ffn_norm_w", "ffn_norm.weight"), ("ffn_norm_b", "ffn_norm.bias"),
               ("fc1_w", "ffn.fc1.weight"), ("fc1_b", "ffn.fc1.bias"),
               ("fc2_w", "ffn.fc2.weight"), ("fc2_b", "ffn.fc2.bias"))


def _dims_of(pe) -> dict:
    """Shapes read off a VAESemanticEncoder module."""
    a0 = pe.encoder.layers[0].attn
    return dict(latent_dim=pe.ds_proj.in_channels, patch=pe.patch_size, hidden=pe.encoder.hidden_size,
                heads=a0.num_heads, ffn=pe.encoder.layers[0].ffn.fc1.out_features,
                n_layers=len(pe.encoder.layers), out_dim=pe.out_proj.out_features,
                ln_eps=float(pe.encoder.layers[0].attn_norm.eps))


class HipPatchEncoder:
    """FlashPatchEncoder (flash_patch_encoder.py:35-139) on the HIP library."""

    def __init__(self, patch_encoder=None, *, max_batch: int, max_seq_len: int, device, dtype=torch.bfloat16,
                 weights: dict | None = None, dims: dict | None = None):
        if dtype != torch.bfloat16:
            raise RuntimeError("HipPatchEncoder runs in bf16")
        if patch_encoder is not None:
            weights = patch_encoder.state_dict()
            dims = _dims_of(patch_encoder)
        if weights is None or dims is None:
            raise RuntimeError("HipPatchEncoder needs the patch encoder module (or weights and dims)")
        self.device = torch.device(device)
        self.dims = dict(dims)
        self.out_ds_rate = dims["patch"] // 2
        self.max_batch, self.cap = int(max_batch), int(max_seq_len)
        lib = _lib.lib()
        keep = {k: v.detach().to(self.device, torch.bfloat16).contiguous() for k, v in weights.items()
                if not k.endswith("inv_freq")}
        L = dims["n_layers"]
        layers = (_lib.DfhPatchEncLayerWeights * L)()
        for l in range(L):
            for f, k in _LAYER_KEYS:
                setattr(layers[l], f, _lib.ptr(keep[f"encoder.layers.{l}.{k}"]))
        w = _lib.DfhPatchEncWeights(ds_w=_lib.ptr(keep["ds_proj.weight"]), ds_b=_lib.ptr(keep["ds_proj.bias"]),
                                    in_w=_lib.ptr(keep["in_proj.weight"]), in_b=_lib.ptr(keep["in_proj.bias"]),
                                    out_w=_lib.ptr(keep["out_proj.weight"]), out_b=_lib.ptr(keep["out_proj.bias"]),
                                    layers=layers)
        cfg = _lib.DfhPatchEncConfig(latent_dim=dims["latent_dim"], patch=dims["patch"], hidden=dims["hidden"],
                                     heads=dims["heads"], ffn=dims["ffn"], n_layers=L, out_dim=dims["out_dim"],
                                     max_batch=self.max_batch, capacity=self.cap,
                                     ln_eps=dims.get("ln_eps", 1e-5))
        h = _lib.vp()
        torch.cuda.synchronize(self.device)  # the weight copies read `keep`
        _lib.check(lib.dfh_patchenc_create(C.byref(cfg), C.byref(w), C.byref(h)), "dfh_patchenc_create")
        self._h = h

    def _rows(self, rows) -> torch.Tensor:
        r = torch.as_tensor(rows, dtype=torch.int32)
        return r.to(self.device).contiguous()

    def reset_rows(self, rows) -> None:
        """Length 0 and a zero conv tail for these cache rows (flash_patch_encoder.py:64-69)."""
        r = self._rows(rows)
        _lib.check(_lib.lib().dfh_patchenc_reset_rows(self._h, _lib.ptr(r), r.numel(), _lib.stream_ptr()),
                   "dfh_patchenc_reset_rows")

    @torch.no_grad()
    def decode_patch(self, latent_patches: torch.Tensor, rows) -> torch.Tensor:
        """latent_patches [n, patch, latent_dim] (denormalised), rows int32 [n]
        distinct cache rows -> embeddings [n, 1, out_dim] bf16; each row's
        history advances by out_ds_rate (flash_patch_encoder.py:103-139)."""
        d = self.dims
        if latent_patches.dim() != 3 or tuple(latent_patches.shape[1:]) != (d["patch"], d["latent_dim"]):
            raise RuntimeError(f"decode_patch: patches {tuple(latent_patches.shape)}, expected "
                               f"[n, {d['patch']}, {d['latent_dim']}]")
        x = latent_patches.to(self.device, torch.bfloat16).contiguous()
        r = self._rows(rows)
        n = x.shape[0]
        if r.numel() != n:
            raise RuntimeError(f"decode_patch: {n} patches but {r.numel()} rows")
        out = torch.empty(n, d["out_dim"], device=self.device, dtype=torch.bfloat16)
        _lib.check(_lib.lib().dfh_patchenc_decode(self._h, _lib.ptr(x), x.stride(0), _lib.ptr(r), n, _lib.ptr(out),
                                                  _lib.stream_ptr()), "dfh_patchenc_decode")
        return out.view(n, 1, d["out_dim"])

    def lengths(self) -> tuple[list[int], bool]:
        """Every row's history length and whether a decode passed a row's
        capacity since the last call (synchronizes)."""
        ln = (C.c_int * self.max_batch)()
        ov = C.c_int(0)
        _lib.check(_lib.lib().dfh_patchenc_lengths(self._h, ln, C.byref(ov)), "dfh_patchenc_lengths")
        return list(ln), bool(ov.value)

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.load_library().dfh_patchenc_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
