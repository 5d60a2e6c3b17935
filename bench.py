"""Benchmark of the MeanFlow FM/DiT head on one MI355X.

Workload (one "step" = one full MeanFlow NFE=4 solve over one batch): 64
concurrent requests, context lengths U{64..1024}, 16 latent rows x 64-d each,
12-block DiT (hidden 1024, 16 heads x 64, MLP 4096) in bf16, random-init
weights N(0, 0.02), contexts N(0,1), noise N(0,1), g_cond = 0.

Prints one JSON line:
  value        DiT GEMM TFLOP/s = executed GEMM FLOPs per solve / wall-per-solve:
               NFE * [11 * 2*M*(4H^2 + 2HF) + 2*M*2H^2 + 2*N*P*(2H^2 + 2HF)],
               M = sum(c_i + 16) unpadded rows; the last block projects K|V over
               every row and Q, O and the MLP over the N*P latent rows only, the
               rows the caller keeps (reference_equivalent_tflops counts 12 full
               blocks instead)
  roofline     the dominant GEMM (largest total time) timed with dispatch-packet
               HIP events inside the timed region
  cpu_baseline the oracle's float32 DiT on the host cores over a bounded
               sample of the same workload (first k requests, full NFE=4 solve)

    python bench.py [--gpus 1] [--steps 10] [--warmup 3]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
PEAK_INT8_TOPS = 5000.0        # MI355X dense int8 MFMA
FRAME_S = 0.04                 # one latent frame = 1920 samples at 48 kHz


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "pmc_hbm_traffic_dit_kernels_meanflow_nfe4_64req.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pmc_traffic(role: str):
    """HBM bytes per launch of ``role`` from the committed FETCH_SIZE/WRITE_SIZE
    summary of this workload (two rocprofv3 --pmc runs, copy-calibrated), or None."""
    found = {}
    try:
        for line in open(TRAFFIC_PROFILE):
            f = line.split()
            if len(f) == 3 and f[0] == "traffic_bytes_per_launch":
                found[f[1]] = int(f[2])
    except OSError:
        return None
    return found.get(role)


def host_cpu():
    """The host's CPU as this process sees it: os.cpu_count(), the CPUs it may run
    on (affinity), the cgroup CPU quota, lscpu's model name, and the thread count
    used for the baseline (affinity, capped by the quota: more threads than the
    quota only time-slice)."""
    import subprocess
    info = {"os_cpu_count": os.cpu_count()}
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    info["affinity_cpus"] = aff
    quota = None
    try:
        q, per = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = int(q) / int(per)
    except (OSError, ValueError):
        pass
    info["cgroup_cpu_quota"] = quota
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    info["lscpu_model"] = model
    info["omp_num_threads_env"] = os.environ.get("OMP_NUM_THREADS")
    threads = aff if quota is None else max(1, min(aff, int(quota)))
    info["threads_used"] = threads
    return info


def cpu_dit_block(threads: int, warmup: int = 3, runs: int = 10):
    """One DiT block on the host (hidden 1024, 16 x 64 heads, MLP 4096) in
    float32 over 64 context + 16 latent rows, t = dt = 0.25, seed 0 (the oracle's
    DiTBlock, the computation tests/golden/c1_block.npz pins). Median of ``runs``
    timed runs after ``warmup``; GFLOP/s of the block's GEMMs (25,165,824 FLOP
    per row)."""
    import numpy as np
    import torch
    from oracle import dit_ref as R
    torch.set_num_threads(threads)
    cfg = R.DitConfig(hidden=1024, heads=16, ffn=4096, n_blocks=1, latent_dim=64, patch=16)
    W = R.random_dit_weights(cfg, 0)
    rs = np.random.RandomState(0)
    x = torch.from_numpy(rs.standard_normal((1, 80, 1024)).astype(np.float32))
    mask = R.build_fm_attn_mask(64, 80, 16)[None]
    pos = R.build_fm_pos_ids(64, 80, 16)[None]
    t = torch.full((1,), 0.25)
    Rg = R._R("fp32")
    with torch.no_grad():
        c = R.condition(W, cfg, t, t, torch.zeros(1, 1024), Rg)
        h = Rg.linear(x, W["input_layer.weight"], W["input_layer.bias"])
        times = []
        for i in range(warmup + runs):
            t0 = time.perf_counter()
            R.block_forward_padded(W, cfg, 0, h, c, mask, pos, Rg)
            if i >= warmup:
                times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    flops = 25_165_824 * 80
    return {"gflops": round(flops / med / 1e9, 2), "median_ms": round(med * 1e3, 3), "runs": runs,
            "warmup": warmup, "threads": threads, "block_gemm_gflop": round(flops / 1e9, 3)}


def cpu_baseline(cfg, W, lens, hist, noise, budget_s: float, threads: int):
    """Oracle fp32 MeanFlow solve of the first k requests on the host cores."""
    import torch
    from oracle import dit_ref as R
    torch.set_num_threads(threads)
    k = 1
    samples = []
    t_spent = 0.0
    while True:
        sub = hist[:k]
        inp, mask, pos, g = R.pack_fm_inputs(sub, cfg.patch, cfg.hidden)
        t0 = time.perf_counter()
        with torch.no_grad():
            R.meanflow_solve_varlen(W, cfg, sub, g, noise[:k], 4, "fp32")
        dt = time.perf_counter() - t0
        t_spent += dt
        M = sum(L + cfg.patch for L in lens[:k])
        samples.append((k, M, dt))
        log(f"cpu baseline: k={k} M={M} {dt:.2f}s")
        if t_spent + 2.5 * dt > budget_s or k * 2 > len(lens):
            break
        k *= 2
    k, M, dt = samples[-1]
    flops = R.dit_gemm_flops(cfg, M) * 4
    return {
        "value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": (f"oracle float32 MeanFlow NFE=4 solve of the first {k} of the 64 requests "
                   f"(M={M} rows/step) on {threads} host threads, torch {torch.__version__}, "
                   f"mkldnn={torch.backends.mkldnn.is_available()}"),
        "xRT": k * cfg.patch * FRAME_S / dt,
        "seconds": dt,
    }


def w8a8_bench(reps: int = 20):
    """W8A8 linears in isolation at the largest token count of that configuration
    (M = 16384): activation quantisation + i8 MFMA GEMM with fused dequant/bias."""
    import torch
    from nanovllm_dots_amd.int8 import gemm_w8a8, quant_act, quant_weight
    M = 16384
    out = {}
    for K, N in [(1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024)]:
        g = torch.Generator(device="cpu").manual_seed(K + N)
        x = torch.randn(M, K, generator=g).bfloat16().cuda()
        w = (0.02 * torch.randn(N, K, generator=g)).bfloat16().cuda()
        b = torch.zeros(N, device="cuda", dtype=torch.bfloat16)
        wq, sw = quant_weight(w)
        xq, sx = quant_act(x)
        gemm_w8a8(xq, wq, sx, sw, b)
        torch.cuda.synchronize()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        for _ in range(reps):
            xq, sx = quant_act(x)
        e[1].record()
        for _ in range(reps):
            gemm_w8a8(xq, wq, sx, sw, b)
        e[2].record()
        torch.cuda.synchronize()
        q_ms = e[0].elapsed_time(e[1]) / reps
        g_ms = e[1].elapsed_time(e[2]) / reps
        ops = 2 * M * K * N
        out[f"K{K}_N{N}"] = {"gemm_tops": round(ops / g_ms / 1e9, 1),
                             "gemm_frac_int8_peak": round(ops / g_ms / 1e9 / PEAK_INT8_TOPS, 4),
                             "quant_GBps": round(M * K * 3 / q_ms / 1e6, 1),
                             "linear_tops": round(ops / (g_ms + q_ms) / 1e9, 1)}
        log(f"w8a8 K={K} N={N}: gemm {out[f'K{K}_N{N}']['gemm_tops']} TOPS, quant {q_ms*1e3:.1f} us")
    return out


def int8_solve_bench(mf, head, solve, ms_bf16: float, gemm_flops: float, steps: int, out_bf16):
    """The same 64-request solve in W8A8 mode (the reference's quantize_dit_ DiT,
    D/int8_dit.py; reported there as 2x slower than bf16 on A100): every DiT
    linear with min(in, out) >= 512 as int8 x int8 -> int32 with per-token
    activation quantisation and a dequantising epilogue. Latents against the
    bf16 solve's are reported (the cost of W8A8 itself)."""
    import torch
    head.set_int8(True)
    for _ in range(2):
        out = solve()
    torch.cuda.synchronize()
    # per-class times from an evented pass of their own (every launch evented
    # adds dispatch time); the timed solves carry no events
    head.profile(True)
    head.profile_read()
    for _ in range(steps):
        out = solve()
    torch.cuda.synchronize()
    prof = head.profile_read()
    head.profile(False)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        out = solve()
    e1.record()
    torch.cuda.synchronize()
    head.set_int8(False)
    ms = e0.elapsed_time(e1) / steps
    a, b = out.float().reshape(-1, out.shape[-1]), out_bf16.float().reshape(-1, out.shape[-1])
    cos = torch.nn.functional.cosine_similarity(a, b, dim=-1)
    gemm_ms = sum(prof[k][0] for k in ("qkv_gemm", "o_gemm", "fc1_gemm", "fc2_gemm")) / steps
    res = {"ms_per_solve": round(ms, 3), "speedup_vs_bf16": round(ms_bf16 / ms, 3),
           "latent_xRT": round(out.shape[0] * out.shape[1] * FRAME_S / (ms * 1e-3), 1),
           "gemm_tops": round(gemm_flops / (ms * 1e-3) / 1e12, 1),
           "quantise_ms_per_solve": round(prof["quantise"][0] / steps, 3),
           "per_class_ms": {k: round(v[0] / steps, 3) for k, v in prof.items()},
           "latents_vs_bf16_cos_min": round(cos.min().item(), 6)}
    log(f"int8 solve: {res}")
    return res


def power_bench(reps: int = 20):
    """The fc2 GEMM shape (M = 36937, N = 1024, K = 4096, bias epilogue) on two
    schedules (tile 8: 8 waves, 128x64 per wave; tile 9: 4 waves, 128x128 per
    wave in AGPRs), with the bench's N(0,1) / N(0,0.02) operands and with all-zero
    operands: the same instructions and the same bytes moved, only the data
    differs. The gap is the chip's power limit, which lowers the shader clock
    under random bf16 operands (data-dependent MFMA switching)."""
    import torch
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    M, N, K = 36937, 1024, 4096
    g = torch.Generator(device="cpu").manual_seed(7)
    ops = {"random": (torch.randn(M, K, generator=g).bfloat16().cuda(),
                      (0.02 * torch.randn(N, K, generator=g)).bfloat16().cuda())}
    ops["zeros"] = (torch.zeros_like(ops["random"][0]), torch.zeros_like(ops["random"][1]))
    bias = torch.zeros(N, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    ws = torch.zeros(4096 + 256 * 256 * 256, device="cuda", dtype=torch.float32)
    res = {"shape": {"M": M, "N": N, "K": K}, "tflops": {}}
    for tile, name in ((8, "tile8_256x256_8wave"), (9, "tile9_256x256_4wave_agpr")):
        for data, (A, B) in ops.items():
            def call():
                _lib.check(lib.dfh_gemm_bf16_ws(_lib.ptr(A), K, _lib.ptr(B), K, _lib.ptr(out), N, _lib.ptr(bias),
                                                M, N, K, 0, tile, _lib.ptr(ws), ws.numel() * 4, _lib.stream_ptr()))
            for _ in range(3):
                call()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                call()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / reps * 1e3
            res["tflops"][f"{name}_{data}"] = round(2.0 * M * N * K / us / 1e6, 1)
    log(f"power: {res}")
    return res


def kvcache_bench(head, cfg, reps: int = 10, n: int = 4, patches: int = 600):
    """Long-audio cached solve: 4 streams, each with a cached prefix of 600 prior
    patches x 16 rows + 512 context rows (the last of them is the active block's
    hidden row), full 12-block DiT, NFE=4. Returns timings, xRT and the decode
    attention's HBM rate over the cached K/V."""
    import numpy as np
    import torch
    from nanovllm_dots_amd import HipFMCache
    rows = patches * 16 + 512
    L = rows - 1
    H = cfg.hidden
    n_ext = 4  # per-patch extends timed after the solves (16 rows per stream each)
    rs = np.random.RandomState(5)
    hist = torch.from_numpy(rs.standard_normal((n, rows + 16 * n_ext, H)).astype(np.float32)).bfloat16().cuda()
    noise = torch.from_numpy(rs.standard_normal((n, cfg.patch, cfg.latent_dim)).astype(np.float32)).bfloat16().cuda()
    cache = HipFMCache(head, n, rows + 16 * n_ext + cfg.patch + 8, 4)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    cache.extend(hist[:, :L], [L] * n)
    e1.record()
    torch.cuda.synchronize()
    prime_ms = e0.elapsed_time(e1)
    lh = hist[:, L].contiguous()
    for _ in range(2):
        out = cache.solve(lh, noise=noise)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        out = cache.solve(lh, noise=noise)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    # per-kernel-class times from a second, profiled pass (its launches carry timestamps)
    head.profile(True)
    head.profile_read()
    for _ in range(reps):
        out = cache.solve(lh, noise=noise)
    torch.cuda.synchronize()
    prof = head.profile_read()
    head.profile(False)
    assert torch.isfinite(out.float()).all()
    # the engine's per-patch step besides the solve: extend every stream by one patch (16 rows)
    e0.record()
    for k in range(n_ext):
        cache.extend(hist[:, L + 1 + 16 * k: L + 1 + 16 * (k + 1)], [16] * n)
    e1.record()
    torch.cuda.synchronize()
    ext_ms = e0.elapsed_time(e1) / n_ext
    attn_ms, attn_n = prof["attention"]
    kv_bytes_launch = n * 2 * (L + 1 + cfg.patch) * H * 2       # one layer's K and V, all streams
    gbps = kv_bytes_launch / (attn_ms / attn_n * 1e-3) / 1e9
    prime_flops = cfg.n_blocks * 2 * (4 * H * H + 2 * H * cfg.ffn) * (4 * n * L)
    res = {"streams": n, "prefix_rows": L, "nfe": 4, "solve_ms": round(ms, 3),
           "latent_xRT": round(n * cfg.patch * FRAME_S / (ms * 1e-3), 1),
           "kv_bytes_per_step": kv_bytes_launch * cfg.n_blocks,
           "decode_attn_us_per_layer": round(attn_ms / attn_n * 1e3, 2),
           "decode_attn_GBps": round(gbps, 1), "decode_attn_frac_hbm": round(gbps / PEAK_HBM_GBS, 4),
           "prime_ms": round(prime_ms, 2), "prime_tflops": round(prime_flops / (prime_ms * 1e-3) / 1e12, 1),
           "kernel_ms_per_solve": {k: round(v[0] / reps, 3) for k, v in prof.items() if v[1]},
           "extend_16_rows_ms": round(ext_ms, 3)}
    log(f"kvcache: {res}")
    cache.close()
    return res


def paged_bench(reps: int = 20):
    """Paged KV-cache attention of the LLM backbone (Qwen2.5-1.5B: 12 query heads,
    2 KV heads, head_dim 128, 256-token pages), 64 sequences x 4096 cached keys in
    shuffled pages: decode (1 new token each) and a 4-token append. Called through
    the C ABI with every argument built once, so the time is the kernels'.
    HBM-bound: the compulsory bytes are every K and V row once, plus q and out."""
    import ctypes as C
    import torch
    from nanovllm_dots_amd import _lib
    lib = _lib.lib()
    B, H, Hkv, hd, bs, L = 64, 12, 2, 128, 256, 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    pages = B * L // bs
    kc = torch.randn(pages, bs, Hkv, hd, device=dev, generator=g).bfloat16()
    vc = torch.randn(pages, bs, Hkv, hd, device=dev, generator=g).bfloat16()
    bt = torch.randperm(pages, device=dev, generator=g).to(torch.int32).view(B, L // bs).contiguous()
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    res = {"config": "64 seqs x 4096 keys in shuffled 256-token pages, 12/2 heads, head_dim 128"}
    for name, lq in (("decode", 1), ("append4", 4)):
        q = torch.randn(B * lq, H, hd, device=dev, generator=g).bfloat16()
        out = torch.empty_like(q)
        cu_q = torch.arange(0, (B + 1) * lq, lq, dtype=torch.int32, device=dev)
        a = _lib.DfhPagedAttnArgs(batch=B, num_heads=H, num_kv_heads=Hkv, head_dim=hd, max_seqlen_q=lq,
                                  max_seqlen_k=L, q=_lib.ptr(q), q_stride=H * hd, cu_seqlens_q=_lib.ptr(cu_q),
                                  k=_lib.ptr(kc), v=_lib.ptr(vc), kv_stride=Hkv * hd, cu_seqlens_k=None,
                                  seqlens_k=_lib.ptr(lens), block_table=_lib.ptr(bt), block_table_stride=L // bs,
                                  block_size=bs, out=_lib.ptr(out), out_stride=H * hd, softmax_scale=hd ** -0.5,
                                  causal=1, workspace=None, workspace_bytes=0)
        ws = torch.empty(lib.dfh_paged_attention_workspace(C.byref(a)) // 4, device=dev)
        a.workspace, a.workspace_bytes = _lib.ptr(ws), ws.numel() * 4
        st = _lib.stream_ptr()
        for _ in range(3):
            _lib.check(lib.dfh_paged_attention(C.byref(a), st), "dfh_paged_attention")
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            lib.dfh_paged_attention(C.byref(a), st)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        nbytes = 2 * B * L * Hkv * hd * 2 + 2 * 2 * B * lq * H * hd
        res[name] = {"us_per_call": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1),
                     "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nbytes}
    log(f"paged: {res}")
    return res


def varlen_bench(mf, hist, noise_d, g_d, ref_out, reps: int = 5):
    """The same 64-request solve from per-request history tensors (dfh_meanflow_solve_varlen):
    no padded [N,T,H] batch, [N,T,T] mask or pos_ids exists."""
    import torch
    dev = noise_d.device
    seqs = [h.to(dev, torch.bfloat16) for h in hist]
    lens = [h.shape[0] for h in hist]
    out = mf.solve_varlen(sequences=seqs, lengths=lens, g_cond=g_d, noise=noise_d)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        out = mf.solve_varlen(sequences=seqs, lengths=lens, g_cond=g_d, noise=noise_d)
    e1.record()
    torch.cuda.synchronize()
    res = {"ms_per_solve": round(e0.elapsed_time(e1) / reps, 4),
           "bit_identical_to_padded": bool(torch.equal(out, ref_out))}
    log(f"varlen: {res}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--requests", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-w8a8", action="store_true")
    ap.add_argument("--no-kvcache", action="store_true")
    ap.add_argument("--no-paged", action="store_true")
    ap.add_argument("--no-power", action="store_true")
    ap.add_argument("--no-int8", action="store_true")
    ap.add_argument("--w8a8-only", action="store_true",
                    help="run only the W8A8 linears leg (M = 16384, four (K, N) shapes) and print its record")
    ap.add_argument("--kvcache-only", action="store_true",
                    help="run only the KV-cached solve leg (4 streams x 10,111 cached rows) and print its record")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run a device copy of this size first (HBM counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU (--gpus 1): the FM head would shard requests across "
              "GPUs with no collective on the hot path, and the multi-GPU path is not built.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from oracle import dit_ref as R
    from nanovllm_dots_amd import FMSpec, HipFMHead, HipMeanflow

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.w8a8_only:
        print(json.dumps({"w8a8_m16384": w8a8_bench()}), flush=True)
        return
    if args.calib_copy_mib:
        src = torch.empty(args.calib_copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cfg = R.DitConfig(hidden=1024, heads=16, ffn=4096, n_blocks=12, latent_dim=64, patch=16)
    log("generating weights / inputs")
    W = R.random_dit_weights(cfg, args.seed)
    if args.kvcache_only:
        print(json.dumps({"kvcache_4x10111": kvcache_bench(HipFMHead(FMSpec.of(cfg), W, device=dev), cfg)}),
              flush=True)
        return
    lens, hist, noise = R.synthetic_requests(args.requests, 64, 1024, cfg, seed=args.seed,
                                             regime="bf16")
    inp, _, pos, g = R.pack_fm_inputs(hist, cfg.patch, cfg.hidden)
    n, T = inp.shape[:2]
    M = sum(L + cfg.patch for L in lens)
    head = HipFMHead(FMSpec.of(cfg), W, device=dev)
    mf = HipMeanflow(None, num_steps=4, dit=object(), head=head)
    inp_d = inp.to(dev, torch.bfloat16)
    pos_d = pos.to(dev)
    g_d = g.to(dev, torch.bfloat16)
    noise_d = noise.to(dev, torch.bfloat16)
    del inp

    def solve():
        return mf(input_sequence=inp_d, attn_mask=None, pos_ids=pos_d, g_cond=g_d, noise=noise_d)

    log(f"warmup x{args.warmup} (n={n}, T={T}, M={M})")
    for _ in range(args.warmup):
        out = solve()
    torch.cuda.synchronize()

    # Kernel classes: every launch carries dispatch-packet events in a pass of
    # its own (untimed; an evented launch costs a few microseconds of dispatch),
    # which also names the dominant GEMM role for the roofline.
    Hd, Fd = cfg.hidden, cfg.ffn
    per_launch = {"qkv_gemm": 2 * M * Hd * 3 * Hd, "o_gemm": 2 * M * Hd * Hd,
                  "fc1_gemm": 2 * M * Hd * Fd, "fc2_gemm": 2 * M * Fd * Hd}
    n_prof = max(2, args.steps // 2)
    head.profile(True)
    head.profile_read()
    for _ in range(n_prof):
        out = solve()
    torch.cuda.synchronize()
    classes = head.profile_read()
    head.profile(False)
    dom = max(per_launch, key=lambda k: classes[k][0])

    # timed region: K solves; a sample of the dominant role's launches carries
    # events (every 7th: 7 is prime to the 11 full-row blocks of a pass, so the
    # sample cycles through them; each evented launch costs about 12 us of
    # dispatch around it, about 0.55 ms per solve when all 44 carry events)
    head.profile(True, classes=(dom,), every=7)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        out = solve()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = e0.elapsed_time(e1)
    prof = head.profile_read()
    head.profile(False)
    ms = ms_total / args.steps
    log(f"timed: {ms:.3f} ms/solve (host wall {wall / args.steps * 1e3:.3f} ms)")
    assert torch.isfinite(out.float()).all()

    H, F = cfg.hidden, cfg.ffn
    ref_gemm_flops = R.dit_gemm_flops(cfg, M) * 4
    # GEMM FLOPs the solve executes: the last block projects K|V over every row
    # and Q, O and the MLP over the n*P latent rows only (latent tail)
    NP = n * cfg.patch
    gemm_flops = 4 * (R.dit_gemm_flops(cfg, M) - M * 2 * (2 * H * H + 2 * H * F)
                      + NP * 2 * (2 * H * H + 2 * H * F))
    tflops = gemm_flops / (ms * 1e-3) / 1e12
    xrt = n * cfg.patch * FRAME_S / (ms * 1e-3)
    # compulsory HBM bytes per launch: A, W, outputs (+ residual read for gate-residual)
    algo_bytes = {"qkv_gemm": 2 * (M * H + 3 * H * H + 3 * M * H),
                  "o_gemm": 2 * (M * H + H * H + 2 * M * H),
                  "fc1_gemm": 2 * (M * H + F * H + M * F),
                  "fc2_gemm": 2 * (M * F + F * H + 2 * M * H)}
    role_ms = {k: classes[k][0] for k in per_launch}
    dom_ms, dom_n = prof[dom]  # the timed region's launches of the dominant role
    avg_ms = dom_ms / max(dom_n, 1)
    achieved = per_launch[dom] / (avg_ms * 1e-3) / 1e12
    breakdown = {k: {"ms_per_solve": v[0] / n_prof, "launches_per_solve": v[1] / n_prof}
                 for k, v in classes.items()}
    gemm_ms = sum(role_ms.values()) / n_prof
    gemm_flops_big = 4 * (cfg.n_blocks - 1) * (per_launch["qkv_gemm"] + per_launch["o_gemm"]
                                               + per_launch["fc1_gemm"] + per_launch["fc2_gemm"])
    log("per-class ms/solve: " + ", ".join(f"{k}={v['ms_per_solve']:.3f}" for k, v in breakdown.items()))

    i8 = None if args.no_int8 else int8_solve_bench(mf, head, solve, ms, gemm_flops, max(3, args.steps // 2), out)
    vl = varlen_bench(mf, hist, noise_d, g_d, out)
    pg = None if args.no_paged else paged_bench()
    w8 = None if args.no_w8a8 else w8a8_bench()
    kvc = None if args.no_kvcache else kvcache_bench(head, cfg)
    pw = None if args.no_power else power_bench()

    cpu = c1 = host = None
    if not args.no_cpu:
        host = host_cpu()
        log(f"host cpu: {host}")
        c1 = cpu_dit_block(host["threads_used"])
        log(f"cpu one-block fp32: {c1}")
        cpu = cpu_baseline(cfg, W, lens, hist, noise, args.cpu_budget, host["threads_used"])

    rec = {
        "metric": "DiT GEMM TFLOPS (% MFMA peak) + latent xRT at 64 streams, NFE=4",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded RandomState; random-init N(0,0.02) weights)",
        "config": {"workload": "meanflow_nfe4_solve_64req_ctx64-1024", "requests": n,
                   "ctx_range": [64, 1024], "patch": cfg.patch, "latent_dim": cfg.latent_dim,
                   "hidden": H, "heads": cfg.heads, "ffn": F, "blocks": cfg.n_blocks, "nfe": 4,
                   "rotary": cfg.rotary, "qk_norm": cfg.qk_norm, "qkv_bias": cfg.qkv_bias,
                   "tokens_per_step_unpadded": M, "padded_T": T},
        "pct_mfma_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "gemm_flops_per_solve": gemm_flops,
        "reference_gemm_flops_per_solve": ref_gemm_flops,
        "reference_equivalent_tflops": round(ref_gemm_flops / (ms * 1e-3) / 1e12, 2),
        "latent_xRT": round(xrt, 1),
        # the four full-size GEMM classes only (the latent tail's small GEMMs are timed apart)
        "gemm_only_tflops": (round(gemm_flops_big / (gemm_ms * 1e-3) / 1e12, 2) if gemm_ms > 0 else None),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": pmc_traffic(dom),
                     "traffic_unit": "bytes/launch", "algorithmic_bytes": algo_bytes[dom],
                     "avg_launch_ms": round(avg_ms, 5), "flops_per_launch": per_launch[dom]},
        "kernel_breakdown": breakdown,
        "w8a8_m16384": w8,
        "kvcache_4x10111": kvc,
        "varlen_solve": vl,
        "llm_paged_attention": pg,
        "gemm_power_limit_fc2_shape": pw,
        "int8_w8a8_solve": i8,
        "cpu_baseline": ({k: (round(v, 5) if isinstance(v, float) else v) for k, v in cpu.items()
                          if k in ("value", "unit", "cores", "kind", "sample")} if cpu else None),
        "cpu_xRT": round(cpu["xRT"], 4) if cpu else None,
        "cpu_dit_block_80rows_fp32": c1,
        "cpu_host": dict(host, torch=torch.__version__, mkldnn=torch.backends.mkldnn.is_available())
        if host else None,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
