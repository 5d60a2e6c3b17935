"""``fm_accel="hip"``: the MeanFlow FM/DiT head on hand-written gfx950 kernels.

Drop-in callables for the reference's accelerator slots
(nanovllm_dots/models/dots/engine.py:125-185, :615-633, :711-723):

* ``HipMeanflow(core, num_steps=4, dit=None)`` — same constructor and
  ``__call__`` signature as ``GraphedMeanflow`` (graphed_meanflow.py:26-60):
  one whole solve per call, returns a fresh ``[N, P, latent_dim]`` bf16 tensor,
  draws noise on the torch RNG outside the kernels when none is given, raises
  ``RuntimeError`` on an NFE mismatch. Unlike the graph it replaces it never
  captures, so a new (N, T) shape costs nothing beyond a workspace grow.
* ``HipDiT(dit)`` — the per-forward ``vfp`` callable
  (``vfp(*, x, timesteps, duration, attn_mask, pos_ids, g_cond) -> [B, T, ld]``,
  batched_fm.py:120-121).
* ``batched_meanflow(core, *, ..., vfp=None)`` — same signature as
  batched_fm.py:82-93.

Weights are read once from the DiT module's state dict (names of
native/dit.py / native/layers.py) plus ``core.coordinate_proj``, and packed by
the library (fused QKV, one adaLN matrix for every block).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class FMSpec:
    """Shape of the DiT head (see include/dots_fm.h DfhConfig)."""
    hidden: int
    heads: int
    ffn: int
    n_blocks: int
    latent_dim: int
    patch: int
    qkv_bias: bool = False
    qk_norm: str = "none"       # "none" | "LayerNorm" | "RMSNorm"
    rotary: bool = True
    rotary_theta: float = 50000.0
    freq_dim: int = 256
    meanflow: bool = True
    ln_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @classmethod
    def of(cls, obj) -> "FMSpec":
        """From any object with the same attribute names (duck-typed)."""
        return cls(**{f: getattr(obj, f) for f in cls.__dataclass_fields__})

    @classmethod
    def from_modules(cls, dit, core) -> "FMSpec":
        """From a reference DiT module (native/dit.py:111-133) and its core."""
        blk = dit.blocks[0]
        attn = blk.attn
        qn = type(attn.q_norm).__name__
        rot = bool(getattr(attn, "rotary_bias", False))
        return cls(
            hidden=dit.input_layer.out_features, heads=attn.num_heads,
            ffn=blk.ffn.fc1.out_features, n_blocks=len(dit.blocks),
            latent_dim=core.latent_dim, patch=core.latent_patch_size,
            qkv_bias=attn.q_proj.bias is not None,
            qk_norm={"Identity": "none"}.get(qn, qn), rotary=rot,
            rotary_theta=float(getattr(attn.rotary, "_theta", 50000.0)) if rot else 50000.0,
            freq_dim=dit.time_embedder.frequency_embedding_size,
            meanflow=getattr(dit, "duration_embedder", None) is not None,
            ln_eps=float(blk.norm1.eps))


def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """RotaryEmbedding.inv_freq (native/layers.py:110-113), float32 on the host."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))


def timestep_freqs(dim: int, max_period: float = 10000.0) -> torch.Tensor:
    """TimestepEmbedder frequencies (native/dit.py:35-38), float32 on the host."""
    half = dim // 2
    return torch.exp(-math.log(max_period) * torch.arange(start=0, end=half, dtype=torch.float32) / half)


def meanflow_grid(num_steps: int, dtype=torch.bfloat16):
    """``linspace(0, 1, nfe+1)`` in the solver dtype and its bf16 step sizes
    (batched_fm.py:113-116)."""
    times = torch.linspace(0.0, 1.0, num_steps + 1, dtype=dtype)
    ts = [float(times[s]) for s in range(num_steps)]
    dts = [float(times[s + 1] - times[s]) for s in range(num_steps)]
    return ts, dts


_QKN = {"none": 0, "LayerNorm": 1, "RMSNorm": 2}


class HipFMHead:
    """Owns one library handle: packed weights + a growable workspace."""

    def __init__(self, spec: FMSpec, weights: dict[str, torch.Tensor], device=None,
                 inv_freq: torch.Tensor | None = None, int8: bool = False):
        self.lib = _lib.lib()
        self.spec = spec
        self.device = torch.device(device if device is not None else "cuda")
        s = spec
        inv = (inv_freq.float().cpu() if inv_freq is not None
               else rope_inv_freq(s.head_dim, s.rotary_theta)).contiguous()
        tf = timestep_freqs(s.freq_dim).contiguous()
        self._inv = (C.c_float * inv.numel())(*inv.tolist())
        self._tf = (C.c_float * tf.numel())(*tf.tolist())
        cfg = _lib.DfhConfig(
            hidden=s.hidden, heads=s.heads, head_dim=s.head_dim, ffn=s.ffn, n_blocks=s.n_blocks,
            latent_dim=s.latent_dim, patch=s.patch, freq_dim=s.freq_dim, qkv_bias=int(s.qkv_bias),
            qk_norm=_QKN[s.qk_norm], rotary=int(s.rotary), meanflow=int(s.meanflow),
            ln_eps=float(s.ln_eps), rope_inv_freq=C.cast(self._inv, C.POINTER(C.c_float)),
            temb_freqs=C.cast(self._tf, C.POINTER(C.c_float)))
        h = _lib.vp()
        with torch.cuda.device(self.device):
            _lib.check(self.lib.dfh_create(C.byref(cfg), C.byref(h)), "dfh_create")
        self.handle = h
        self.int8 = False
        self.set_weights(weights)
        if int8 and not self.int8:
            self.set_int8(True)

    # -- weights --------------------------------------------------------------
    def int8_linear_names(self) -> list[str]:
        """The DiT linears quantize_dit_ turns into W8A8 (min(in, out) >= 512,
        D/int8_dit.py:71-85), in the order the library packs them."""
        s = self.spec
        names = ["input_layer", "time_embedder.mlp.2"] + (["duration_embedder.mlp.2"] if s.meanflow else [])
        for l in range(s.n_blocks):
            p = f"blocks.{l}."
            names += [p + n for n in ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj", "ffn.fc1",
                                      "ffn.fc2", "adaLN_modulation.1")]
        return names + ["output_layer.adaLN_modulation.1"]

    @staticmethod
    def _split_int8(W: dict[str, torch.Tensor]):
        """A quantize_dit_-ed state dict holds, per W8A8 linear, an int8 weight
        (Int8DynamicLinear: ``Wt_int8`` [in, out]; HipInt8Linear: ``W_int8``
        [out, in]) and ``w_scale`` instead of ``weight``. Returns the state dict
        with a bf16 stand-in ``weight`` (q * s, used only if W8A8 is switched
        off) and {linear: (int8 [out, in], scale [out])}."""
        W = dict(W)
        q8 = {}
        for k in list(W):
            for suffix, transpose in ((".Wt_int8", True), (".W_int8", False)):
                if k.endswith(suffix):
                    name = k[: -len(suffix)]
                    q = W.pop(k)
                    q = (q.t() if transpose else q).contiguous()
                    sc = W.pop(name + ".w_scale").float().contiguous()
                    q8[name] = (q, sc)
                    if name + ".weight" not in W:
                        W[name + ".weight"] = (q.float() * sc[:, None]).to(torch.bfloat16)
        return W, q8

    def set_weights(self, W: dict[str, torch.Tensor]) -> None:
        s = self.spec
        keep = []
        W, q8 = self._split_int8(W)

        def dev(name, required=True):
            t = W.get(name)
            if t is None:
                if required:
                    raise KeyError(f"missing DiT parameter {name!r}")
                return None
            t = t.detach().to(device=self.device, dtype=torch.bfloat16).contiguous()
            keep.append(t)
            return _lib.ptr(t)

        blocks = (_lib.DfhBlockWeights * s.n_blocks)()
        for l in range(s.n_blocks):
            p = f"blocks.{l}."
            b = blocks[l]
            for nm in ("q", "k", "v"):
                setattr(b, f"{nm}_w", dev(p + f"attn.{nm}_proj.weight"))
                setattr(b, f"{nm}_b", dev(p + f"attn.{nm}_proj.bias", s.qkv_bias))
            if s.qk_norm != "none":
                b.q_norm_w = dev(p + "attn.q_norm.weight")
                b.k_norm_w = dev(p + "attn.k_norm.weight")
                if s.qk_norm == "LayerNorm":
                    b.q_norm_b = dev(p + "attn.q_norm.bias")
                    b.k_norm_b = dev(p + "attn.k_norm.bias")
            b.o_w, b.o_b = dev(p + "attn.o_proj.weight"), dev(p + "attn.o_proj.bias")
            b.fc1_w, b.fc1_b = dev(p + "ffn.fc1.weight"), dev(p + "ffn.fc1.bias")
            b.fc2_w, b.fc2_b = dev(p + "ffn.fc2.weight"), dev(p + "ffn.fc2.bias")
            b.ada_w = dev(p + "adaLN_modulation.1.weight")
            b.ada_b = dev(p + "adaLN_modulation.1.bias")
        w = _lib.DfhWeights(
            input_w=dev("input_layer.weight"), input_b=dev("input_layer.bias"),
            t_w0=dev("time_embedder.mlp.0.weight"), t_b0=dev("time_embedder.mlp.0.bias"),
            t_w2=dev("time_embedder.mlp.2.weight"), t_b2=dev("time_embedder.mlp.2.bias"),
            d_w0=dev("duration_embedder.mlp.0.weight", s.meanflow),
            d_b0=dev("duration_embedder.mlp.0.bias", s.meanflow),
            d_w2=dev("duration_embedder.mlp.2.weight", s.meanflow),
            d_b2=dev("duration_embedder.mlp.2.bias", s.meanflow),
            final_ada_w=dev("output_layer.adaLN_modulation.1.weight"),
            final_ada_b=dev("output_layer.adaLN_modulation.1.bias"),
            final_w=dev("output_layer.linear.weight"), final_b=dev("output_layer.linear.bias"),
            coord_w=dev("coordinate_proj.weight"), coord_b=dev("coordinate_proj.bias"),
            blocks=C.cast(blocks, C.POINTER(_lib.DfhBlockWeights)))
        with torch.cuda.device(self.device):
            _lib.check(self.lib.dfh_set_weights(self.handle, C.byref(w), _lib.stream_ptr()),
                       "dfh_set_weights")
        del keep
        self.int8 = False
        if q8:
            self.set_int8(True, q8)

    def set_int8(self, enable: bool, q8: dict | None = None) -> None:
        """W8A8 solve (the reference's quantize_dit_ DiT, D/int8_dit.py): every
        linear of int8_linear_names() runs as Int8DynamicLinear. Its int8 weights
        come from q8 ({linear: (int8 [out, in], scale [out])}, as a quantized
        module holds them) or, without q8, are quantised from the bf16 weights
        as Int8DynamicLinear(lin) does. A partly quantised DiT is refused."""
        if not enable:
            _lib.check(self.lib.dfh_set_int8(self.handle, 0, None, _lib.stream_ptr()), "dfh_set_int8")
            self.int8 = False
            return
        s = self.spec
        names = self.int8_linear_names()
        arg = None
        keep = []
        if q8:
            missing = [n for n in names if n not in q8]
            if missing:
                raise RuntimeError(f"partly quantised DiT: no int8 weight for {missing[:4]}")

            def lin(*parts):
                q = torch.cat([q8[p][0] for p in parts]).to(self.device, torch.int8).contiguous()
                sc = torch.cat([q8[p][1] for p in parts]).to(self.device, torch.float32).contiguous()
                keep.extend((q, sc))
                return _lib.DfhInt8Linear(_lib.ptr(q), _lib.ptr(sc))

            L = s.n_blocks
            qkv, o, fc1, fc2 = ((_lib.DfhInt8Linear * L)() for _ in range(4))
            for l in range(L):
                p = f"blocks.{l}."
                qkv[l] = lin(p + "attn.q_proj", p + "attn.k_proj", p + "attn.v_proj")
                o[l], fc1[l], fc2[l] = lin(p + "attn.o_proj"), lin(p + "ffn.fc1"), lin(p + "ffn.fc2")
            arg = _lib.DfhInt8Weights(
                input=lin("input_layer"), t_mlp2=lin("time_embedder.mlp.2"),
                d_mlp2=lin("duration_embedder.mlp.2") if s.meanflow else _lib.DfhInt8Linear(None, None),
                ada=lin(*[f"blocks.{l}.adaLN_modulation.1" for l in range(L)], "output_layer.adaLN_modulation.1"),
                qkv=C.cast(qkv, C.POINTER(_lib.DfhInt8Linear)), o=C.cast(o, C.POINTER(_lib.DfhInt8Linear)),
                fc1=C.cast(fc1, C.POINTER(_lib.DfhInt8Linear)), fc2=C.cast(fc2, C.POINTER(_lib.DfhInt8Linear)))
        with torch.cuda.device(self.device):
            _lib.check(self.lib.dfh_set_int8(self.handle, 1, C.byref(arg) if arg is not None else None,
                                             _lib.stream_ptr()), "dfh_set_int8")
        del keep
        self.int8 = True

    # -- entry points -----------------------------------------------------------
    def solve(self, input_sequence, pos_ids, g_cond, noise, num_steps: int, *, strict=False):
        s = self.spec
        n, T, H = input_sequence.shape
        self._check_inputs(input_sequence, pos_ids, g_cond)
        if noise.shape != (n, s.patch, s.latent_dim):
            raise RuntimeError(f"noise shape {tuple(noise.shape)} != {(n, s.patch, s.latent_dim)}")
        inp = input_sequence.to(torch.bfloat16).contiguous()
        pos = pos_ids.to(torch.float32).contiguous()
        g = g_cond.to(torch.bfloat16).contiguous() if g_cond is not None else None
        nz = noise.to(torch.bfloat16).contiguous()
        out = torch.empty((n, s.patch, s.latent_dim), device=inp.device, dtype=torch.bfloat16)
        ts, dts = meanflow_grid(num_steps)
        tg = (C.c_float * num_steps)(*ts)
        dg = (C.c_float * num_steps)(*dts)
        args = _lib.DfhSolveArgs(n=n, total_len=T, num_steps=num_steps, input_sequence=_lib.ptr(inp),
                                 pos_ids=_lib.ptr(pos), g_cond=_lib.ptr(g), noise=_lib.ptr(nz),
                                 out=_lib.ptr(out), t_grid=tg, dt_grid=dg)
        st = _lib.stream_ptr()
        _lib.check(self.lib.dfh_meanflow_solve(self.handle, C.byref(args), st), "dfh_meanflow_solve")
        if strict:
            self._raise_input_status(st)
        return out

    def solve_varlen(self, sequences, lengths, g_cond, noise, num_steps: int, *, strict=False):
        """One solve over requests as the engine holds them: request i's history is
        the first ``lengths[i]`` rows of ``sequences[i]`` (``[L, H]`` or ``[1, L, H]``
        bf16 on the GPU, e.g. ``fm_sequence``). No padded batch, mask or pos_ids is
        built (engine.py:635-688); the result equals :meth:`solve` on the padded
        batch of the same requests."""
        s = self.spec
        n = len(sequences)
        if n == 0 or len(lengths) != n:
            raise RuntimeError(f"need one length per sequence, got {n} sequences and {len(lengths)} lengths")
        rows = [q[0] if q.dim() == 3 else q for q in sequences]
        stride = None
        for q, L in zip(rows, lengths):
            if q.dim() != 2 or q.shape[1] != s.hidden or q.dtype != torch.bfloat16 or not q.is_cuda:
                raise RuntimeError(f"each sequence must be a bf16 [L, {s.hidden}] GPU tensor, got "
                                   f"{tuple(q.shape)} {q.dtype} on {q.device}")
            if not 1 <= int(L) <= q.shape[0]:
                raise RuntimeError(f"history length {int(L)} outside [1, {q.shape[0]}]")
            if stride is None:
                stride = q.stride(0)
            if q.stride(1) != 1 or q.stride(0) != stride or q.data_ptr() % 16 or stride % 8:
                # one row stride for every request, 16-B aligned rows
                stride = None
                break
        if stride is None:
            rows = [q[:int(L)].contiguous() for q, L in zip(rows, lengths)]
            stride = s.hidden
        if noise.shape != (n, s.patch, s.latent_dim):
            raise RuntimeError(f"noise shape {tuple(noise.shape)} != {(n, s.patch, s.latent_dim)}")
        dev = rows[0].device
        ptrs = torch.tensor([q.data_ptr() for q in rows], dtype=torch.int64).to(dev)
        lens = torch.tensor([int(L) for L in lengths], dtype=torch.int32).to(dev)
        g = g_cond.reshape(n, s.hidden).to(torch.bfloat16).contiguous() if g_cond is not None else None
        nz = noise.to(torch.bfloat16).contiguous()
        out = torch.empty((n, s.patch, s.latent_dim), device=dev, dtype=torch.bfloat16)
        ts, dts = meanflow_grid(num_steps)
        tg = (C.c_float * num_steps)(*ts)
        dg = (C.c_float * num_steps)(*dts)
        args = _lib.DfhVarlenSolveArgs(n=n, max_hist=max(int(L) for L in lengths), num_steps=num_steps,
                                       hist_rows=_lib.ptr(ptrs), hist_len=_lib.ptr(lens), row_stride=stride,
                                       g_cond=_lib.ptr(g), noise=_lib.ptr(nz), out=_lib.ptr(out),
                                       t_grid=tg, dt_grid=dg)
        st = _lib.stream_ptr()
        _lib.check(self.lib.dfh_meanflow_solve_varlen(self.handle, C.byref(args), st),
                   "dfh_meanflow_solve_varlen")
        if strict:
            self._raise_input_status(st)
        return out

    def forward(self, x, timesteps, duration, pos_ids, g_cond, *, strict=False):
        s = self.spec
        n, T, H = x.shape
        self._check_inputs(x, pos_ids, g_cond)
        xx = x.to(torch.bfloat16).contiguous()
        pos = pos_ids.to(torch.float32).contiguous()
        g = g_cond.to(torch.bfloat16).contiguous() if g_cond is not None else None
        tv = timesteps.reshape(-1).to(device=xx.device, dtype=torch.float32).expand(n).contiguous()
        dv = None
        if duration is not None and s.meanflow:
            dv = duration.reshape(-1).to(device=xx.device, dtype=torch.float32).expand(n).contiguous()
        out = torch.empty((n, T, s.latent_dim), device=xx.device, dtype=torch.bfloat16)
        args = _lib.DfhForwardArgs(n=n, total_len=T, x=_lib.ptr(xx), timesteps=_lib.ptr(tv),
                                   duration=_lib.ptr(dv), pos_ids=_lib.ptr(pos), g_cond=_lib.ptr(g),
                                   out=_lib.ptr(out))
        st = _lib.stream_ptr()
        _lib.check(self.lib.dfh_dit_forward(self.handle, C.byref(args), st), "dfh_dit_forward")
        if strict:
            self._raise_input_status(st)
        return out

    def reserve(self, n: int, total_len: int, num_steps: int = 4) -> None:
        _lib.check(self.lib.dfh_reserve(self.handle, n, total_len, num_steps, _lib.stream_ptr()),
                   "dfh_reserve")

    def set_ksplit(self, enable: bool) -> None:
        """K-split of each GEMM's last partial round of tiles (on by default)."""
        _lib.check(self.lib.dfh_set_ksplit(self.handle, int(enable)), "dfh_set_ksplit")

    def set_ln_quant(self, enable: bool) -> None:
        """int8 mode: quantise QKV's and fc1's input rows inside LayerNorm+modulate
        (on by default; bit-identical to the separate quantiser pass)."""
        _lib.check(self.lib.dfh_set_ln_quant(self.handle, int(enable)), "dfh_set_ln_quant")

    def set_latent_tail(self, enable: bool) -> None:
        """Last block of a solve on the latent rows only (on by default): the
        caller keeps v[:, -P:] (batched_fm.py:122-124), so only those rows'
        attention, O projection and MLP are computed there."""
        _lib.check(self.lib.dfh_set_latent_tail(self.handle, int(enable)), "dfh_set_latent_tail")

    def profile(self, enable: bool, classes=None, every: int = 1) -> None:
        """Dispatch-packet events on the launches of ``classes`` (names from
        PROFILE_CLASSES; None: all) while ``enable``: launches 0, every,
        2*every, ... of each class from this call on; read with profile_read()."""
        mask = 0xFFFFFFFF if classes is None else sum(1 << self.PROFILE_CLASSES.index(c) for c in classes)
        _lib.check(self.lib.dfh_profile_classes(self.handle, mask, int(every)), "dfh_profile_classes")
        _lib.check(self.lib.dfh_profile_enable(self.handle, int(enable)), "dfh_profile_enable")

    PROFILE_CLASSES = ("qkv_gemm", "o_gemm", "fc1_gemm", "fc2_gemm", "attention", "ln_modulate", "other",
                       "latent_tail", "quantise")

    def profile_read(self) -> dict[str, tuple[float, int]]:
        k = len(self.PROFILE_CLASSES)
        ms = (C.c_double * k)()
        cnt = (C.c_long * k)()
        _lib.check(self.lib.dfh_profile_read(self.handle, ms, cnt, k), "dfh_profile_read")
        return {name: (ms[i], cnt[i]) for i, name in enumerate(self.PROFILE_CLASSES)}

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.dfh_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- helpers ---------------------------------------------------------------
    def _check_inputs(self, x, pos_ids, g_cond):
        s = self.spec
        if x.dim() != 3 or x.shape[2] != s.hidden:
            raise RuntimeError(f"input must be [N, T, {s.hidden}], got {tuple(x.shape)}")
        n, T, _ = x.shape
        if not x.is_cuda:
            raise RuntimeError("input must be on the GPU")
        if T <= s.patch:
            raise RuntimeError(f"total_len {T} must exceed the latent patch {s.patch}")
        if pos_ids.shape != (n, T):
            raise RuntimeError(f"pos_ids shape {tuple(pos_ids.shape)} != {(n, T)}")
        if g_cond is not None and g_cond.reshape(n, -1).shape[1] != s.hidden:
            raise RuntimeError("g_cond must be [N, hidden]")

    def _raise_input_status(self, st):
        flags = C.c_int(0)
        _lib.check(self.lib.dfh_input_status(self.handle, C.byref(flags), st), "dfh_input_status")
        if flags.value & 1:
            raise RuntimeError("the inputs do not describe a valid FM layout (history length "
                               "c = pos_ids[i, T-P], or hist_len[i], must be an integer in [1, T-P])")
        if flags.value & 2:
            raise RuntimeError("a history row base is not 16-byte aligned")


def _weights_from_modules(dit, core) -> dict[str, torch.Tensor]:
    W = dict(dit.state_dict())
    W["coordinate_proj.weight"] = core.coordinate_proj.weight
    W["coordinate_proj.bias"] = core.coordinate_proj.bias
    return W


class HipMeanflow:
    """Whole-solve MeanFlow on the HIP kernels; a drop-in for GraphedMeanflow."""

    def __init__(self, core, *, num_steps: int = 4, dit=None, warmup: int = 0, head: HipFMHead = None,
                 strict: bool = False):
        self.core = core
        self.nfe = num_steps
        self.dit = dit if dit is not None else getattr(core, "velocity_field_predictor", None)
        self.strict = strict
        if head is None:
            spec = FMSpec.from_modules(self.dit, core)
            inv = None
            if spec.rotary:
                inv = self.dit.blocks[0].attn.rotary.inv_freq
            head = HipFMHead(spec, _weights_from_modules(self.dit, core),
                             device=next(self.dit.parameters()).device, inv_freq=inv)
        self.head = head
        self.latent_dim = head.spec.latent_dim
        self.patch = head.spec.patch

    @torch.no_grad()
    def __call__(self, *, input_sequence, attn_mask, pos_ids, g_cond, num_steps=None, noise=None):
        if num_steps is not None and num_steps != self.nfe:
            raise RuntimeError(f"HipMeanflow built for nfe={self.nfe}, got {num_steps}.")
        n = input_sequence.shape[0]
        if noise is None:
            noise = torch.randn((n, self.patch, self.latent_dim), device=input_sequence.device,
                                dtype=input_sequence.dtype)
        return self.head.solve(input_sequence, pos_ids, g_cond, noise, self.nfe, strict=self.strict)


    @torch.no_grad()
    def solve_varlen(self, *, sequences, lengths, g_cond=None, num_steps=None, noise=None):
        """The whole solve straight from per-request histories (``fm_sequence``,
        ``fm_seq_len``), in place of ``_pack_fm_inputs`` + ``__call__``
        (engine.py:635-688, :713-724). Same noise and NFE rules as ``__call__``."""
        if num_steps is not None and num_steps != self.nfe:
            raise RuntimeError(f"HipMeanflow built for nfe={self.nfe}, got {num_steps}.")
        n = len(sequences)
        if noise is None:
            noise = torch.randn((n, self.patch, self.latent_dim), device=sequences[0].device,
                                dtype=torch.bfloat16)
        return self.head.solve_varlen(sequences, lengths, g_cond, noise, self.nfe, strict=self.strict)


class HipDiT:
    """The per-forward ``vfp`` callable: DiT.forward on the HIP kernels."""

    def __init__(self, dit=None, core=None, *, head: HipFMHead = None, strict: bool = False):
        if head is None:
            spec = FMSpec.from_modules(dit, core)
            inv = dit.blocks[0].attn.rotary.inv_freq if spec.rotary else None
            head = HipFMHead(spec, _weights_from_modules(dit, core),
                             device=next(dit.parameters()).device, inv_freq=inv)
        self.head = head
        self.strict = strict

    @torch.no_grad()
    def __call__(self, *, x, timesteps, duration=None, attn_mask=None, pos_ids=None, g_cond=None,
                 **_kwargs):
        if pos_ids is None:
            raise RuntimeError("HipDiT needs pos_ids (the FM layout is read from them)")
        return self.head.forward(x, timesteps, duration, pos_ids, g_cond, strict=self.strict)


@torch.no_grad()
def batched_meanflow(core, *, input_sequence, attn_mask, pos_ids, g_cond, num_steps: int = 4,
                     noise=None, vfp=None):
    """batched_fm.batched_meanflow with the HIP head. ``vfp=None`` runs the whole
    solve in one library call (a HipMeanflow cached on ``core``); a ``HipDiT``
    vfp runs the per-step loop of batched_fm.py:113-125 around it."""
    n = input_sequence.size(0)
    P = core.latent_patch_size
    if noise is None:
        noise = torch.randn((n, P, core.latent_dim), device=input_sequence.device,
                            dtype=input_sequence.dtype)
    if vfp is None:
        mf = getattr(core, "_hip_meanflow", None)
        if mf is None or mf.nfe != num_steps:
            mf = HipMeanflow(core, num_steps=num_steps)
            core._hip_meanflow = mf
        return mf(input_sequence=input_sequence, attn_mask=attn_mask, pos_ids=pos_ids, g_cond=g_cond,
                  num_steps=num_steps, noise=noise)
    if not isinstance(vfp, HipDiT):
        raise TypeError("batched_meanflow(fm_accel='hip') takes vfp=None or a HipDiT")
    latent_start = input_sequence.size(1) - P
    times = torch.linspace(0.0, 1.0, num_steps + 1, device=input_sequence.device,
                           dtype=input_sequence.dtype)
    z = noise
    for step in range(num_steps):
        t = times[step].expand(n)
        dt = (times[step + 1] - times[step]).expand(n)
        zp = core.coordinate_proj(z)
        z_c = input_sequence.clone()
        z_c[:, latent_start:] = zp
        vt = vfp(x=z_c, timesteps=t, duration=dt, attn_mask=attn_mask, pos_ids=pos_ids, g_cond=g_cond)
        z = z + vt[:, latent_start:] * dt.view(-1, 1, 1)
    return z


class HipFMCache:
    """Prefix K/V cache + cached MeanFlow solve for ``n_streams`` streams.

    The MeanFlow counterpart of the reference's per-timestep FM cache
    (nanovllm_dots/models/dots/cached_fm.py:82-197, written there for the CFG
    flow-matching DiT): ``extend`` appends history rows to every stream's
    prefix at all ``num_steps`` timesteps in one batched pass; ``solve`` runs the
    NFE-step solve of the active rows (last hidden row + latent patch) against
    the cache, equal to a full-recompute solve of prefix + last hidden row.
    """

    def __init__(self, head: HipFMHead, n_streams: int, capacity: int, num_steps: int = 4):
        self.head = head
        self.lib = head.lib
        self.n = n_streams
        self.nfe = num_steps
        h = _lib.vp()
        _lib.check(self.lib.dfh_kvcache_create(head.handle, n_streams, capacity, num_steps, C.byref(h)),
                   "dfh_kvcache_create")
        self.cache = h
        ts, dts = meanflow_grid(num_steps)
        self._tg = (C.c_float * num_steps)(*ts)
        self._dg = (C.c_float * num_steps)(*dts)

    @property
    def lengths(self) -> list[int]:
        arr = (C.c_int * self.n)()
        _lib.check(self.lib.dfh_kvcache_lengths(self.cache, arr), "dfh_kvcache_lengths")
        return list(arr)

    def reset(self) -> None:
        _lib.check(self.lib.dfh_kvcache_reset(self.cache, _lib.stream_ptr()), "dfh_kvcache_reset")

    def extend(self, rows: torch.Tensor, counts, g_cond=None) -> None:
        """rows: [n, m_max, H] (FM sequence space); counts[i] rows of stream i."""
        s = self.head.spec
        if rows.dim() != 3 or rows.shape[0] != self.n or rows.shape[2] != s.hidden:
            raise RuntimeError(f"rows must be [{self.n}, m, {s.hidden}], got {tuple(rows.shape)}")
        r = rows.to(torch.bfloat16).contiguous()
        g = g_cond.to(torch.bfloat16).contiguous() if g_cond is not None else None
        cnt = (C.c_int * self.n)(*[int(x) for x in counts])
        _lib.check(self.lib.dfh_kvcache_extend(self.cache, _lib.ptr(r), r.shape[1], cnt, _lib.ptr(g),
                                               self._tg, self._dg, _lib.stream_ptr()), "dfh_kvcache_extend")

    def solve(self, last_hidden: torch.Tensor, g_cond=None, noise=None) -> torch.Tensor:
        s = self.head.spec
        lh = last_hidden.reshape(self.n, s.hidden).to(torch.bfloat16).contiguous()
        if noise is None:
            noise = torch.randn((self.n, s.patch, s.latent_dim), device=lh.device, dtype=torch.bfloat16)
        nz = noise.to(torch.bfloat16).contiguous()
        g = g_cond.to(torch.bfloat16).contiguous() if g_cond is not None else None
        out = torch.empty((self.n, s.patch, s.latent_dim), device=lh.device, dtype=torch.bfloat16)
        _lib.check(self.lib.dfh_kvcache_solve(self.cache, _lib.ptr(lh), _lib.ptr(g), _lib.ptr(nz), _lib.ptr(out),
                                              self._tg, self._dg, _lib.stream_ptr()), "dfh_kvcache_solve")
        return out

    def close(self) -> None:
        if getattr(self, "cache", None):
            self.lib.dfh_kvcache_destroy(self.cache)
            self.cache = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
