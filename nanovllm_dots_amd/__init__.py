"""nanovllm_dots_amd — the MeanFlow FM/DiT head of nanovllm_dots on MI355X.

Hand-written gfx950 HIP kernels (libdotsfm.so, C ABI in include/dots_fm.h)
behind the reference's accelerator entry points (``fm_accel="hip"``).
"""
from .hip_meanflow import (FMSpec, HipDiT, HipFMCache, HipFMHead, HipMeanflow, batched_meanflow,  # noqa: F401
                           meanflow_grid, rope_inv_freq, timestep_freqs)

from .patch_encoder import HipPatchEncoder  # noqa: F401

__all__ = ["HipPatchEncoder", "FMSpec", "HipDiT", "HipFMCache", "HipFMHead", "HipMeanflow", "batched_meanflow", "meanflow_grid",
           "rope_inv_freq", "timestep_freqs"]
