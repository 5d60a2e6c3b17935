// Row and elementwise kernels of the FM/DiT head (HBM-bound; one wave per row).
#include "dfh_device.h"
#include "dfh_kernels.h"
#include "dfh_ops.h"

namespace dfh {

namespace {

// ---------------------------------------------------------------------------
// LayerNorm (no affine, eps) + adaLN modulate, one wave per row.
// DiTBlock.forward / FinalLayer.forward (nanovllm_dots/models/dots/native/dit.py:
// 99-105, 60-63) under bf16 autocast: LN in fp32, (1 + scale) rounded to bf16,
// fp32 product and sum, one rounding to bf16 at the consumer's input.
//
// QO: the row also leaves as the int8 input of the next W8A8 linear (q, sx),
// exactly what the per-token quantiser makes of the bf16 row
// (D/int8_dit.py:57-58; the operations of quant_rows_kernel); out may then be
// null (no bf16 row stored).
template <int VPT, bool QO>  // values per lane = H / 64, multiple of 4
__global__ void __launch_bounds__(256)
ln_modulate_kernel(const uint16_t* __restrict__ x, long ldx, uint16_t* __restrict__ out, long ldo,
                   const uint16_t* __restrict__ shift, const uint16_t* __restrict__ scale,
                   long ld_mod, const int* __restrict__ row_req, const int* __restrict__ row_map,
                   int rows, const int* __restrict__ M_dev, int H, float eps, int8_t* __restrict__ q,
                   long ldq, float* __restrict__ sx) {
  // 16-B accesses (8 values) where the row splits evenly, else 8-B
  constexpr int W = VPT % 8 == 0 ? 8 : 4;
  constexpr int NJ = VPT / W;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nrows = M_dev ? *M_dev : rows;
  if (r >= nrows) return;
  const int src = row_map ? row_map[r] : r;
  const int req = row_req[src];
  const uint16_t* xp = x + (long)src * ldx;
  const uint16_t* shp = shift + (long)req * ld_mod;
  const uint16_t* scp = scale + (long)req * ld_mod;
  // the row and its request's shift / scale all in flight before the reductions
  float v[VPT], sh[VPT], sc[VPT];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = (j * 64 + lane) * W;
    if constexpr (W == 8) {
      const uint4 xq = *reinterpret_cast<const uint4*>(xp + col);
      const uint4 hq = *reinterpret_cast<const uint4*>(shp + col);
      const uint4 cq = *reinterpret_cast<const uint4*>(scp + col);
      unpack4(make_uint2(xq.x, xq.y), v + 8 * j);
      unpack4(make_uint2(xq.z, xq.w), v + 8 * j + 4);
      unpack4(make_uint2(hq.x, hq.y), sh + 8 * j);
      unpack4(make_uint2(hq.z, hq.w), sh + 8 * j + 4);
      unpack4(make_uint2(cq.x, cq.y), sc + 8 * j);
      unpack4(make_uint2(cq.z, cq.w), sc + 8 * j + 4);
    } else {
      unpack4(*reinterpret_cast<const uint2*>(xp + col), v + 4 * j);
      unpack4(*reinterpret_cast<const uint2*>(shp + col), sh + 4 * j);
      unpack4(*reinterpret_cast<const uint2*>(scp + col), sc + 4 * j);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) s += v[j];
  const float mean = wave_sum(s) / (float)H;
  float s2 = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const float d = v[j] - mean;
    s2 += d * d;
  }
  const float var = wave_sum(s2) / (float)H;
  const float rstd = rsqrtf(var + eps);
  float y[VPT];
#pragma unroll
  for (int t = 0; t < VPT; ++t) {
    const float ln = mul_rn(v[t] - mean, rstd);
    const float onep = rbf(1.0f + sc[t]);
    y[t] = add_rn(mul_rn(ln, onep), sh[t]);
  }
  if (!QO || out) {
    uint16_t* op = out + (long)r * ldo;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = (j * 64 + lane) * W;
      if constexpr (W == 8) {
        const uint2 lo = pack4(y[8 * j], y[8 * j + 1], y[8 * j + 2], y[8 * j + 3]);
        const uint2 hi2 = pack4(y[8 * j + 4], y[8 * j + 5], y[8 * j + 6], y[8 * j + 7]);
        *reinterpret_cast<uint4*>(op + col) = make_uint4(lo.x, lo.y, hi2.x, hi2.y);
      } else {
        *reinterpret_cast<uint2*>(op + col) = pack4(y[4 * j], y[4 * j + 1], y[4 * j + 2], y[4 * j + 3]);
      }
    }
  }
  if constexpr (QO) {
    // the bf16 row's absolute maximum, s = bf16(amax / 127) (at least bf16(1e-8)),
    // then bf16(x / s) from y = RN(1 / s) with one FMA correction, rounded, clamped
    float amax = 0.f;
#pragma unroll
    for (int t = 0; t < VPT; ++t) {
      y[t] = rbf(y[t]);
      amax = fmaxf(amax, fabsf(y[t]));
    }
    amax = wave_max(amax);
    float sr = rbf(__fdiv_rn(amax, 127.0f));
    sr = fmaxf(sr, rbf(1e-8f));
    if (lane == 0) sx[r] = sr;
    const float yi = __fdiv_rn(1.0f, sr);
    int8_t* qp = q + (long)r * ldq;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = (j * 64 + lane) * W;
      uint32_t packed[W / 4] = {};
#pragma unroll
      for (int t = 0; t < W; ++t) {
        const float xv = y[W * j + t];
        const float q0 = mul_rn(xv, yi);
        const float q1 = __builtin_fmaf(__builtin_fmaf(-sr, q0, xv), yi, q0);  // RN(x / s)
        float vq = rintf(rbf(q1));
        vq = fminf(fmaxf(vq, -127.f), 127.f);
        packed[t >> 2] |= ((uint32_t)(uint8_t)(int8_t)(int)vq) << (8 * (t & 3));
      }
      if constexpr (W == 8) *reinterpret_cast<uint2*>(qp + col) = make_uint2(packed[0], packed[1]);
      else *reinterpret_cast<uint32_t*>(qp + col) = packed[0];
    }
  }
}

// ---------------------------------------------------------------------------
// Request layout. Padded inputs: c_i = pos_ids[i, T-P] (the first latent row's
// position equals the history length, native/model.py:77-87). Varlen inputs:
// c_i = lens[i]. A length outside [1, T-P] sets err bit 0 and is clamped into
// it (varlen: to 1, so no more than the first row of that request is read).
// One workgroup of up to 1024 threads, one thread per request.
__global__ void __launch_bounds__(1024)
fm_layout_kernel(const float* __restrict__ pos_ids, const int* __restrict__ lens, int n, int T, int P,
                 int* __restrict__ cu_rows, int* __restrict__ cu_vt, int* __restrict__ hist_len,
                 int* __restrict__ counts, int* __restrict__ err, AttnSeq* __restrict__ seqs,
                 AttnSeq* __restrict__ tail_seqs, int* __restrict__ tail_req, int* __restrict__ tail_pos) {
  __shared__ int s_rows[1024], s_vt[1024];
  const int i = threadIdx.x;
  int c = 0;
  if (i < n) {
    bool bad;
    if (lens) {
      c = lens[i];
      bad = c < 1 || c > T - P;
    } else {
      const float pv = pos_ids[(long)i * T + (T - P)];
      c = (int)pv;
      bad = !(pv >= 1.0f) || c > T - P || (float)c != pv;
    }
    if (bad) {
      atomicOr(err, 1);
      c = lens ? 1 : (c < 1 ? 1 : (c > T - P ? T - P : c));
    }
    hist_len[i] = c;
  }
  const int Ti = i < n ? c + P : 0;
  s_rows[i] = Ti;
  s_vt[i] = (Ti + 7) & ~7;
  __syncthreads();
  // inclusive Hillis-Steele scan
  for (int o = 1; o < 1024; o <<= 1) {
    int a = i >= o ? s_rows[i - o] : 0;
    int b = i >= o ? s_vt[i - o] : 0;
    __syncthreads();
    s_rows[i] += a;
    s_vt[i] += b;
    __syncthreads();
  }
  if (i < n) {
    cu_rows[i + 1] = s_rows[i];
    cu_vt[i + 1] = s_vt[i];
    // request i: rows [r0, r0 + c + P); history causal below c - 1
    const int r0 = s_rows[i] - Ti, v0 = s_vt[i] - ((Ti + 7) & ~7);
    seqs[i] = AttnSeq{r0, r0, v0, 0, Ti, c - 1, Ti, r0};
    // the P latent queries alone, output to compact rows i*P .. i*P + P - 1; and
    // the request of each compact row
    if (tail_seqs) tail_seqs[i] = AttnSeq{r0, r0, v0, c, Ti, c - 1, Ti, i * P - c};
    if (tail_req)
      for (int j = 0; j < P; ++j) tail_req[i * P + j] = i;
    if (tail_pos)
      for (int j = 0; j < P; ++j) tail_pos[i * P + j] = c + j;
  }
  if (i == 0) {
    cu_rows[0] = 0;
    cu_vt[0] = 0;
    counts[0] = s_rows[n - 1];           // M: packed rows
    counts[1] = s_vt[n - 1];             // V^T columns used
  }
}

// Padded [N, T, H] (or per-request history rows src_rows[i] + r * src_stride,
// latent slots zero) -> packed rows; builds row tables. One wave per padded row.
// A history base that is not 16-B aligned sets err bit 1; its rows are zeroed.
__global__ void __launch_bounds__(256)
fm_gather_kernel(const uint16_t* __restrict__ inp, const uint16_t* const* __restrict__ src_rows,
                 long src_stride, int n, int T, int P, int H,
                 const int* __restrict__ cu_rows, const int* __restrict__ cu_vt,
                 const int* __restrict__ hist_len, uint16_t* __restrict__ seq, int* __restrict__ row_req,
                 int* __restrict__ row_pos, int* __restrict__ vt_col, int* __restrict__ patch_rows,
                 int* __restrict__ err) {
  const int lane = threadIdx.x & 63;
  const long pr = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pr >= (long)n * T) return;
  const int i = (int)(pr / T), r = (int)(pr % T);
  const int c = hist_len[i];
  int local;
  if (r < c) local = r;
  else if (r >= T - P) local = c + (r - (T - P));
  else return;  // padding gap
  const int dst = cu_rows[i] + local;
  if (lane == 0) {
    row_req[dst] = i;
    row_pos[dst] = local;
    vt_col[dst] = cu_vt[i] + local;
    if (local >= c) patch_rows[i * P + (local - c)] = dst;
  }
  const uint16_t* sp = inp + pr * H;
  if (src_rows) {
    const uint16_t* base = src_rows[i];
    sp = local < c && ((uintptr_t)base & 15) == 0 ? base + (long)local * src_stride : nullptr;
    if (local < c && !sp && lane == 0) atomicOr(err, 2);
  }
  uint16_t* dp = seq + (long)dst * H;
  for (int col = lane * 8; col < H; col += 64 * 8)
    *reinterpret_cast<uint4*>(dp + col) = sp ? *reinterpret_cast<const uint4*>(sp + col) : make_uint4(0u, 0u, 0u, 0u);
}

// packed [M, D] rows -> padded [n, T, D]; rows of the padding gap are zero-filled.
__global__ void unpack_rows_kernel(const uint16_t* __restrict__ src, int n, int T, int P, int D,
                                   const int* __restrict__ cu_rows, const int* __restrict__ hist_len,
                                   uint16_t* __restrict__ dst) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;  // over n*T*D/4
  const long total = (long)n * T * (D / 4);
  if (idx >= total) return;
  const long pr = idx / (D / 4);
  const int col = (int)(idx % (D / 4)) * 4;
  const int i = (int)(pr / T), r = (int)(pr % T);
  const int c = hist_len[i];
  int local = -1;
  if (r < c) local = r;
  else if (r >= T - P) local = c + (r - (T - P));
  uint2 v = make_uint2(0u, 0u);
  if (local >= 0) v = *reinterpret_cast<const uint2*>(src + (long)(cu_rows[i] + local) * D + col);
  *reinterpret_cast<uint2*>(dst + pr * D + col) = v;
}

// RoPE tables: cos/sin of pos * inv_freq[d] in fp32 (native/layers.py:124-134), [max_pos, hd/2]
// Layout (half = 32): groups of 32 positions; within a group, for each
// g = d / 8, the 32 positions' pairs of 16-B chunks (d % 8 < 4, d % 8 >= 4):
// float index (((p / 32) * 4 + g) * 64 + (p % 32) * 2 + (d / 4) % 2) * 4 + d % 4.
// The QKV epilogue's lane (row p, half hi) needs d = 8g + 4hi + [0, 4), so a
// wave's load of one g over 32 consecutive positions reads 1 KB in one or two
// contiguous pieces.
__global__ void rope_table_kernel(const float* __restrict__ inv_freq, int half, int max_pos,
                                  float* __restrict__ cosv, float* __restrict__ sinv) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= max_pos * half) return;
  const int p = idx / half, d = idx % half;
  const float f = mul_rn((float)p, inv_freq[d]);
  const long o = ((long)((p >> 5) * 4 + (d >> 3)) * 64 + (p & 31) * 2 + ((d >> 2) & 1)) * 4 + (d & 3);
  cosv[o] = cosf(f);
  sinv[o] = sinf(f);
}

// Sinusoidal timestep embedding (native/dit.py:34-43): row r has value tv[r];
// [cos(t*f_k) | sin(t*f_k)] rounded to bf16 (the next Linear's input).
// Timestep values come from device memory (tv non-null) or by value (tvh).
__global__ void temb_kernel(const float* __restrict__ tv, TimeVals tvh, int rows,
                            const float* __restrict__ freqs, int half, int dim,
                            uint16_t* __restrict__ out) {
  const int r = blockIdx.x;
  if (r >= rows) return;
  const float t = tv ? tv[r] : tvh.v[r];
  for (int k = threadIdx.x; k < dim; k += blockDim.x) {
    float e = 0.f;
    if (k < half) e = cosf(mul_rn(t, freqs[k]));
    else if (k < 2 * half) e = sinf(mul_rn(t, freqs[k - half]));
    out[(long)r * dim + k] = f2bf(e);
  }
}

// y = bf16(silu(x)) elementwise over n values
__global__ void silu_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = f2bf(silu_f(bf2f(x[i])));
}

// c[s, i] = bf16(bf16(T[s] + D[s]) + g[i]);  a[s*N + i] = bf16(silu(c))
// (per_req: timestep row i instead of s, i.e. one timestep per request)
__global__ void condition_kernel(const uint16_t* __restrict__ temb, const uint16_t* __restrict__ demb,
                                 const uint16_t* __restrict__ g, int S, int N, int H, int per_req,
                                 uint16_t* __restrict__ c_out, uint16_t* __restrict__ a_out) {
  const int row = blockIdx.x;  // s*N + i
  if (row >= S * N) return;
  const int s = row / N, i = row % N;
  const int tr = per_req ? i : s;
  for (int k = threadIdx.x; k < H; k += blockDim.x) {
    float c = bf2f(temb[(long)tr * H + k]);
    if (demb) c = rbf(c + bf2f(demb[(long)tr * H + k]));
    if (g) c = rbf(c + bf2f(g[(long)i * H + k]));
    c_out[(long)row * H + k] = f2bf(c);
    a_out[(long)row * H + k] = f2bf(silu_f(c));
  }
}

// seq[patch_rows[r]] = src[r]   (rows of H bf16)
__global__ void scatter_rows_kernel(const uint16_t* __restrict__ src, const int* __restrict__ rows_idx,
                                    int rows, int H, uint16_t* __restrict__ dst) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint16_t* sp = src + (long)r * H;
  uint16_t* dp = dst + (long)rows_idx[r] * H;
  for (int col = lane * 8; col < H; col += 64 * 8)
    *reinterpret_cast<uint4*>(dp + col) = *reinterpret_cast<const uint4*>(sp + col);
}

// dst[dst_rows[r]] = src[src_rows ? src_rows[r] : r]   (rows of H bf16)
__global__ void gather_rows_kernel(const uint16_t* __restrict__ src, const int* __restrict__ src_rows,
                                   const int* __restrict__ dst_rows, int rows, int H, uint16_t* __restrict__ dst) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint16_t* sp = src + (long)(src_rows ? src_rows[r] : r) * H;
  uint16_t* dp = dst + (long)(dst_rows ? dst_rows[r] : r) * H;
  for (int col = lane * 8; col < H; col += 64 * 8)
    *reinterpret_cast<uint4*>(dp + col) = *reinterpret_cast<const uint4*>(sp + col);
}

// z = bf16(z + bf16(v * dt))  (batched_fm.py:125 in bf16)
__global__ void z_update_kernel(uint16_t* __restrict__ z, const uint16_t* __restrict__ v, float dt,
                                long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) z[i] = f2bf(bf2f(z[i]) + rbf(bf2f(v[i]) * dt));
}

// ---------------------------------------------------------------------------
// Prefix-cache pass tables. Rows of a pass are ordered (timestep k, stream i,
// row r): pass row = k * Mtot + offs[i] + r with Mtot = offs[n]. Stream i's new
// rows r < counts[i] take positions lens[i] + r and land in slab region
// (k, i) = rows/columns [(k*n + i) * cap, +cap). One wave per padded input row.
__global__ void __launch_bounds__(256)
prefix_tables_kernel(const uint16_t* __restrict__ rows_in, long stride_in, int m_max, int H,
                     const int* __restrict__ counts, const int* __restrict__ lens,
                     const int* __restrict__ offs, int n, int S, int cap, uint16_t* __restrict__ seq,
                     int* __restrict__ row_req, int* __restrict__ row_pos, int* __restrict__ c_rows,
                     int* __restrict__ vt_col, AttnSeq* __restrict__ seqs) {
  const int lane = threadIdx.x & 63;
  const long pr = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pr >= (long)S * n * m_max) return;
  const int k = (int)(pr / ((long)n * m_max));
  const int i = (int)((pr / m_max) % n);
  const int r = (int)(pr % m_max);
  const int Mtot = offs[n];
  const int len = lens[i], cnt = counts[i];
  const int base = (k * n + i) * cap;
  if (r == 0 && lane == 0)
    seqs[k * n + i] = AttnSeq{base, base, base, len, len + cnt, len + cnt, len + cnt, k * Mtot + offs[i] - len};
  if (r >= cnt) return;
  const int row = k * Mtot + offs[i] + r;
  if (lane == 0) {
    row_req[row] = k * n + i;
    row_pos[row] = len + r;
    c_rows[row] = base + len + r;
    vt_col[row] = base + len + r;
  }
  const uint16_t* sp = rows_in + (long)i * stride_in + (long)r * H;
  uint16_t* dp = seq + (long)row * H;
  for (int col = lane * 8; col < H; col += 64 * 8)
    *reinterpret_cast<uint4*>(dp + col) = *reinterpret_cast<const uint4*>(sp + col);
}

// Active-pass tables for all S steps: rows (k, i, j), j = 0 the last hidden row
// (position lens[i]), j = 1..P the latent rows; queries of stream i at step k
// are the rows lens[i] .. lens[i] + P of region (k, i), which they all see.
__global__ void active_tables_kernel(const int* __restrict__ lens, int n, int S, int P, int cap,
                                     int* __restrict__ row_req, int* __restrict__ row_pos,
                                     int* __restrict__ c_rows, int* __restrict__ vt_col,
                                     AttnSeq* __restrict__ seqs, int* __restrict__ patch_rows,
                                     int* __restrict__ lh_rows) {
  const int R = 1 + P;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= S * n * R) return;
  const int k = idx / (n * R), i = (idx / R) % n, j = idx % R;
  const int len = lens[i];
  const int base = (k * n + i) * cap;
  row_req[idx] = k * n + i;
  row_pos[idx] = len + j;
  c_rows[idx] = base + len + j;
  vt_col[idx] = base + len + j;
  if (j == 0) seqs[k * n + i] = AttnSeq{base, base, base, len, len + R, 0, len + R, i * R - len};
  if (k == 0) {
    if (j == 0) lh_rows[i] = i * R;
    else patch_rows[i * P + j - 1] = i * R + j;
  }
}

// lens[i] += counts[i]; offs = exclusive prefix sum of counts (offs[n] = total)
__global__ void cache_advance_kernel(int* __restrict__ lens, const int* __restrict__ counts, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) lens[i] += counts[i];
}

}  // namespace

hipError_t prefix_tables(const uint16_t* rows_in, long stride_in, int m_max, int H, const int* counts,
                         const int* lens, const int* offs, int n, int S, int cap, uint16_t* seq, int* row_req,
                         int* row_pos, int* c_rows, int* vt_col, AttnSeq* seqs, hipStream_t s) {
  const long rows = (long)S * n * m_max;
  if (rows <= 0) return hipSuccess;
  if (H % 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(prefix_tables_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, rows_in,
                     stride_in, m_max, H, counts, lens, offs, n, S, cap, seq, row_req, row_pos, c_rows, vt_col,
                     seqs);
  return hipGetLastError();
}

hipError_t active_tables(const int* lens, int n, int S, int P, int cap, int* row_req, int* row_pos,
                         int* c_rows, int* vt_col, AttnSeq* seqs, int* patch_rows, int* lh_rows,
                         hipStream_t s) {
  const int total = S * n * (1 + P);
  hipLaunchKernelGGL(active_tables_kernel, dim3((total + 255) / 256), dim3(256), 0, s, lens, n, S, P, cap,
                     row_req, row_pos, c_rows, vt_col, seqs, patch_rows, lh_rows);
  return hipGetLastError();
}

hipError_t cache_advance(int* lens, const int* counts, int n, hipStream_t s) {
  hipLaunchKernelGGL(cache_advance_kernel, dim3((n + 255) / 256), dim3(256), 0, s, lens, counts, n);
  return hipGetLastError();
}

hipError_t ln_modulate(const uint16_t* x, long ldx, uint16_t* out, long ldo, const uint16_t* shift,
                       const uint16_t* scale, long ld_mod, const int* row_req, const int* row_map,
                       int rows_upper, const int* M_dev, int H, float eps, hipStream_t s, int8_t* q, long ldq,
                       float* sx) {
  if (rows_upper <= 0) return hipSuccess;
  if (H % 256 != 0) return hipErrorInvalidValue;
  if (q ? (!sx || ldq < H || ldq % 8 != 0) : !out) return hipErrorInvalidValue;
  dim3 grid((rows_upper + 3) / 4), block(256);
  switch (H / 64) {
#define DFH_LN(V)                                                                                         \
  case V:                                                                                                \
    if (q)                                                                                               \
      dfh_launch(ln_modulate_kernel<V, true>, grid, block, 0, s, x, ldx, out, ldo, shift, scale, ld_mod, \
                 row_req, row_map, rows_upper, M_dev, H, eps, q, ldq, sx);                               \
    else                                                                                                 \
      dfh_launch(ln_modulate_kernel<V, false>, grid, block, 0, s, x, ldx, out, ldo, shift, scale, ld_mod,\
                 row_req, row_map, rows_upper, M_dev, H, eps, q, ldq, sx);                               \
    break;
    DFH_LN(4)
    DFH_LN(8)
    DFH_LN(16)
    DFH_LN(24)
    DFH_LN(32)
#undef DFH_LN
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t fm_layout(const float* pos_ids, const int* lens, int n, int T, int P, int* cu_rows, int* cu_vt,
                     int* hist_len, int* counts, int* err, AttnSeq* seqs, AttnSeq* tail_seqs, int* tail_req,
                     int* tail_pos, hipStream_t s) {
  if (n <= 0 || n > 1024 || (!pos_ids && !lens)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fm_layout_kernel, dim3(1), dim3(1024), 0, s, pos_ids, lens, n, T, P, cu_rows, cu_vt,
                     hist_len, counts, err, seqs, tail_seqs, tail_req, tail_pos);
  return hipGetLastError();
}

hipError_t fm_gather(const uint16_t* inp, const uint16_t* const* src_rows, long src_stride, int n, int T,
                     int P, int H, const int* cu_rows, const int* cu_vt, const int* hist_len, uint16_t* seq,
                     int* row_req, int* row_pos, int* vt_col, int* patch_rows, int* err, hipStream_t s) {
  const long rows = (long)n * T;
  if (H % 8 != 0 || (!inp && !src_rows) || (src_rows && (src_stride < H || src_stride % 8 != 0)))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(fm_gather_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, inp, src_rows,
                     src_stride, n, T, P, H, cu_rows, cu_vt, hist_len, seq, row_req, row_pos, vt_col,
                     patch_rows, err);
  return hipGetLastError();
}

hipError_t rope_table(const float* inv_freq, int half, int max_pos, float* cosv, float* sinv,
                      hipStream_t s) {
  if (half != 32 || max_pos <= 0) return hipErrorInvalidValue;  // the grouped layout is for head_dim 64
  const int n = half * max_pos;
  hipLaunchKernelGGL(rope_table_kernel, dim3((n + 255) / 256), dim3(256), 0, s, inv_freq, half,
                     max_pos, cosv, sinv);
  return hipGetLastError();
}

hipError_t timestep_embed(const float* tv, const TimeVals& tvh, int rows, const float* freqs, int half,
                          int dim, uint16_t* out, hipStream_t s) {
  if (!tv && rows > kMaxTimeVals) return hipErrorInvalidValue;
  hipLaunchKernelGGL(temb_kernel, dim3(rows), dim3(256), 0, s, tv, tvh, rows, freqs, half, dim, out);
  return hipGetLastError();
}

hipError_t silu_bf16(const uint16_t* x, uint16_t* y, long n, hipStream_t s) {
  hipLaunchKernelGGL(silu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t condition(const uint16_t* temb, const uint16_t* demb, const uint16_t* g, int S, int N,
                     int H, uint16_t* c_out, uint16_t* a_out, hipStream_t s, bool per_request_t) {
  hipLaunchKernelGGL(condition_kernel, dim3(S * N), dim3(256), 0, s, temb, demb, g, S, N, H,
                     per_request_t ? 1 : 0, c_out, a_out);
  return hipGetLastError();
}

hipError_t scatter_rows(const uint16_t* src, const int* rows_idx, int rows, int H, uint16_t* dst,
                        hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (H % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, src, rows_idx, rows,
                     H, dst);
  return hipGetLastError();
}

hipError_t gather_rows(const uint16_t* src, const int* src_rows, const int* dst_rows, int rows, int H,
                       uint16_t* dst, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (H % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, src, src_rows, dst_rows, rows, H,
                     dst);
  return hipGetLastError();
}

hipError_t z_update(uint16_t* z, const uint16_t* v, float dt, long n, hipStream_t s) {
  hipLaunchKernelGGL(z_update_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, z, v, dt, n);
  return hipGetLastError();
}

hipError_t unpack_rows(const uint16_t* src, int n, int T, int P, int D, const int* cu_rows,
                       const int* hist_len, uint16_t* dst, hipStream_t s) {
  if (D % 4 != 0) return hipErrorInvalidValue;
  const long total = (long)n * T * (D / 4);
  hipLaunchKernelGGL(unpack_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, n,
                     T, P, D, cu_rows, hist_len, dst);
  return hipGetLastError();
}

}  // namespace dfh
