// The patch encoder's per-patch decode for n requests at once
// (FlashPatchEncoder.decode_patch, nanovllm_dots/models/dots/flash_patch_encoder.py
// :103-139, over VAESemanticEncoder, native/patch_encoder.py): the row kernels
// it needs besides the GEMMs, the K/V store and the paged attention.
//
// Request i of a call owns cache row rows[i]: its K / V of every layer live at
// rows [rows[i] * cap, rows[i] * cap + len[rows[i]]) of that layer's cache, its
// conv tail (the previous patch's last latent frame) at tail[rows[i]].
#include "dfh_device.h"
#include "dfh_kernels.h"
#include "dfh_ops.h"

namespace dfh {

namespace {

// LayerNorm with affine parameters over H columns, one wave per row: float32
// statistics of the bf16 row, y = (x - mean) * rstd * w + b, one rounding
// (nn.LayerNorm on bf16 tensors, native/patch_encoder.py:34-37).
template <int VPT>  // H / 64
__global__ void __launch_bounds__(256)
ln_affine_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ out, const uint16_t* __restrict__ w,
                 const uint16_t* __restrict__ b, int rows, int H, float eps) {
  constexpr int W = VPT % 8 == 0 ? 8 : 4;
  constexpr int NJ = VPT / W;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint16_t* xp = x + (long)r * H;
  float v[VPT], wv[VPT], bv[VPT];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = (j * 64 + lane) * W;
    if constexpr (W == 8) {
      const uint4 xq = *reinterpret_cast<const uint4*>(xp + col);
      const uint4 wq = *reinterpret_cast<const uint4*>(w + col);
      const uint4 bq = *reinterpret_cast<const uint4*>(b + col);
      unpack4(make_uint2(xq.x, xq.y), v + 8 * j);
      unpack4(make_uint2(xq.z, xq.w), v + 8 * j + 4);
      unpack4(make_uint2(wq.x, wq.y), wv + 8 * j);
      unpack4(make_uint2(wq.z, wq.w), wv + 8 * j + 4);
      unpack4(make_uint2(bq.x, bq.y), bv + 8 * j);
      unpack4(make_uint2(bq.z, bq.w), bv + 8 * j + 4);
    } else {
      unpack4(*reinterpret_cast<const uint2*>(xp + col), v + 4 * j);
      unpack4(*reinterpret_cast<const uint2*>(w + col), wv + 4 * j);
      unpack4(*reinterpret_cast<const uint2*>(b + col), bv + 4 * j);
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
  const float rstd = rsqrtf(wave_sum(s2) / (float)H + eps);
  uint16_t* op = out + (long)r * H;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = (j * 64 + lane) * W;
    float y[W];
#pragma unroll
    for (int t = 0; t < W; ++t) y[t] = (v[W * j + t] - mean) * rstd * wv[W * j + t] + bv[W * j + t];
    if constexpr (W == 8) {
      const uint2 lo = pack4(y[0], y[1], y[2], y[3]), hi = pack4(y[4], y[5], y[6], y[7]);
      *reinterpret_cast<uint4*>(op + col) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    } else {
      *reinterpret_cast<uint2*>(op + col) = pack4(y[0], y[1], y[2], y[3]);
    }
  }
}

// Causal downsample step of request blockIdx.x (native/patch_encoder.py:229-236):
// frames f_0 = tail[rows[i]], f_{1+s} = patch[i][s] (s < P); output token t of
// channel o = bias[o] + sum_c w[o][c][0] f_{2t}[c] + w[o][c][1] f_{2t+1}[c]
// (Conv1d kernel 2, stride 2), float32 sum, one rounding to bf16. The patch's
// last frame becomes the row's new tail after every read of the old one.
__global__ void __launch_bounds__(256)
pe_downsample_kernel(const uint16_t* __restrict__ patch, long patch_stride, const uint16_t* __restrict__ w,
                     const uint16_t* __restrict__ bias, const int* __restrict__ rows, uint16_t* __restrict__ tail,
                     uint16_t* __restrict__ out, int P, int ld) {
  extern __shared__ float frames[];  // [(P + 1) * ld]
  const int i = blockIdx.x, r = rows[i];
  const uint16_t* pp = patch + (long)i * patch_stride;
  for (int e = threadIdx.x; e < (P + 1) * ld; e += blockDim.x)
    frames[e] = bf2f(e < ld ? tail[(long)r * ld + e] : pp[e - ld]);
  __syncthreads();
  const int ods = P / 2;
  for (int e = threadIdx.x; e < ods * ld; e += blockDim.x) {
    const int t = e / ld, o = e % ld;
    const float* f0 = frames + (2 * t) * ld;
    const float* f1 = f0 + ld;
    const uint16_t* wo = w + (long)o * ld * 2;
    float acc = bf2f(bias[o]);
    for (int c = 0; c < ld; ++c) acc += bf2f(wo[2 * c]) * f0[c] + bf2f(wo[2 * c + 1]) * f1[c];
    out[((long)i * ods + t) * ld + o] = f2bf(acc);
  }
  for (int c = threadIdx.x; c < ld; c += blockDim.x) tail[(long)r * ld + c] = pp[(long)(P - 1) * ld + c];
}

// Per-call tables: request i appends its ods new K / V rows at row
// rows[i] * cap + len + j (len = the row's length, j < ods) and attends over
// len + ods keys; queries are rows [i * ods, (i + 1) * ods). A row whose length
// would pass the capacity appends nothing, attends over its cap keys and sets
// *err (the caller checks it); a row index outside [0, max_rows) is replaced by
// row 0 in rows_ok, which every later kernel of the call reads, and sets *err
// too: no access leaves the caches.
__global__ void pe_plan_kernel(const int* __restrict__ rows, const int* __restrict__ len, int n, int ods, int cap,
                               int max_rows, int* __restrict__ rows_ok, int* __restrict__ slots,
                               int* __restrict__ seqlens_k, int* __restrict__ cu_q, int* __restrict__ err) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0) cu_q[n] = n * ods;
  if (i >= n) return;
  int r = rows[i];
  if (r < 0 || r >= max_rows) {
    *err = 1;
    r = 0;
  }
  rows_ok[i] = r;
  const int L = len[r];
  const bool fits = L >= 0 && L + ods <= cap;
  if (!fits) *err = 1;
  seqlens_k[i] = fits ? L + ods : cap;
  cu_q[i] = i * ods;
  for (int j = 0; j < ods; ++j) slots[i * ods + j] = fits ? r * cap + L + j : -1;
}

// after the layers: the rows' lengths advance by ods (not past the capacity)
__global__ void pe_advance_kernel(const int* __restrict__ rows, int* __restrict__ len, int n, int ods, int cap) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int r = rows[i], L = len[r] + ods;
  len[r] = L <= cap ? L : cap;
}

// reset_rows (flash_patch_encoder.py:64-69): length 0 and a zero conv tail. The
// cache rows keep their old K / V: nothing reads keys at or past a row's length.
__global__ void pe_reset_kernel(const int* __restrict__ rows, int n, int max_rows, int* __restrict__ len,
                                uint16_t* __restrict__ tail, int ld) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const int r = rows[i];
  if (r < 0 || r >= max_rows) return;
  if (threadIdx.x == 0) len[r] = 0;
  for (int c = threadIdx.x; c < ld; c += blockDim.x) tail[(long)r * ld + c] = 0;
}

}  // namespace

hipError_t ln_affine(const uint16_t* x, uint16_t* out, const uint16_t* w, const uint16_t* b, int rows, int H,
                     float eps, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (H % 256 != 0) return hipErrorInvalidValue;
  const dim3 grid((rows + 3) / 4), block(256);
  switch (H / 64) {
#define DFH_LNA(V)                                                                       \
  case V:                                                                                \
    dfh_launch(ln_affine_kernel<V>, grid, block, 0, s, x, out, w, b, rows, H, eps);      \
    break;
    DFH_LNA(4)
    DFH_LNA(8)
    DFH_LNA(16)
    DFH_LNA(24)
    DFH_LNA(32)
#undef DFH_LNA
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t pe_downsample(const uint16_t* patch, long patch_stride, const uint16_t* w, const uint16_t* bias,
                         const int* rows, uint16_t* tail, uint16_t* out, int n, int P, int ld, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const size_t lds = (size_t)(P + 1) * ld * sizeof(float);
  if (P % 2 != 0 || lds > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pe_downsample_kernel, dim3(n), dim3(256), lds, s, patch, patch_stride, w, bias, rows, tail,
                     out, P, ld);
  return hipGetLastError();
}

hipError_t pe_plan(const int* rows, const int* len, int n, int ods, int cap, int max_rows, int* rows_ok, int* slots,
                   int* seqlens_k, int* cu_q, int* err, hipStream_t s) {
  hipLaunchKernelGGL(pe_plan_kernel, dim3((n + 63) / 64 > 0 ? (n + 63) / 64 : 1), dim3(64), 0, s, rows, len, n, ods,
                     cap, max_rows, rows_ok, slots, seqlens_k, cu_q, err);
  return hipGetLastError();
}

hipError_t pe_advance(const int* rows, int* len, int n, int ods, int cap, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(pe_advance_kernel, dim3((n + 63) / 64), dim3(64), 0, s, rows, len, n, ods, cap);
  return hipGetLastError();
}

hipError_t pe_reset(const int* rows, int n, int max_rows, int* len, uint16_t* tail, int ld, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(pe_reset_kernel, dim3(n), dim3(64), 0, s, rows, n, max_rows, len, tail, ld);
  return hipGetLastError();
}

}  // namespace dfh
