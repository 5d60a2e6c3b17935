// int8 quantisation kernels of the W8A8 DiT linear (Int8DynamicLinear,
// nanovllm_dots/models/dots/int8_dit.py:34-65). HBM-bound, one wave per row.
//
// Activations (int8_dit.py:57-58) are quantised in the input dtype, bf16: every
// bf16 op is one IEEE float32 op rounded to nearest-even bf16, so
//   s = max(bf16(amax / 127), bf16(1e-8)),  q = clamp(rint(bf16(x / s)), -127, 127)
// with correctly rounded float32 division and round-half-to-even (v_rndne_f32).
// The per-value division x / s uses the row's correctly rounded reciprocal
// y = RN(1/s) and one FMA correction, q = RN(x*y), q' = RN(q + RN(x - s*q)*y),
// which equals RN(x / s) whenever nothing overflows or underflows (Markstein's
// theorem). Only where |x| < 2^-100 can the remainder underflow; such an x / s
// is below 2^-73 and quantises to 0 either way.
// Weights (int8_dit.py:40-45) are quantised in float32:
//   s_w = max(amax / 127, 1e-8),  q = clamp(rint(w / s_w), -127, 127).
#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

// NCH > 0: the row is K = 512 * NCH values, held in registers between the amax
// and the quantise pass (one read of the row); NCH == 0: any K % 8 == 0, read twice
template <int NCH>
__global__ void __launch_bounds__(256)
quant_rows_kernel(const uint16_t* __restrict__ x, long ldx, int8_t* __restrict__ q, long ldq,
                  float* __restrict__ scale, int M, int K, const int* __restrict__ M_dev) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= (M_dev ? *M_dev : M)) return;
  const uint16_t* xp = x + (long)r * ldx;
  constexpr int NR = NCH > 0 ? NCH : 1;
  uint4 row[NR];
  float amax = 0.f;
  auto absmax = [&](const uint4& u) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      amax = fmaxf(amax, fabsf(bf2f((uint16_t)(w[t] & 0xffffu))));
      amax = fmaxf(amax, fabsf(bf2f((uint16_t)(w[t] >> 16))));
    }
  };
  if constexpr (NCH > 0) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) row[j] = *reinterpret_cast<const uint4*>(xp + j * 512 + lane * 8);
#pragma unroll
    for (int j = 0; j < NCH; ++j) absmax(row[j]);
  } else {
    for (int c = lane * 8; c < K; c += 512) absmax(*reinterpret_cast<const uint4*>(xp + c));
  }
  amax = wave_max(amax);
  float s = rbf(__fdiv_rn(amax, 127.0f));
  s = fmaxf(s, rbf(1e-8f));
  if (lane == 0) scale[r] = s;
  const float y = __fdiv_rn(1.0f, s);  // RN(1 / s), once per row
  int8_t* qp = q + (long)r * ldq;
  auto quant8 = [&](const uint4& u, int c) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint16_t h = (uint16_t)((t & 1) ? (w[t >> 1] >> 16) : (w[t >> 1] & 0xffffu));
      const float xv = bf2f(h);
      const float q0 = mul_rn(xv, y);
      const float q1 = __builtin_fmaf(__builtin_fmaf(-s, q0, xv), y, q0);  // RN(x / s)
      float v = rintf(rbf(q1));
      v = fminf(fmaxf(v, -127.f), 127.f);
      packed[t >> 2] |= ((uint32_t)(uint8_t)(int8_t)(int)v) << (8 * (t & 3));
    }
    *reinterpret_cast<uint2*>(qp + c) = make_uint2(packed[0], packed[1]);
  };
  if constexpr (NCH > 0) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) quant8(row[j], j * 512 + lane * 8);
  } else {
    for (int c = lane * 8; c < K; c += 512) quant8(*reinterpret_cast<const uint4*>(xp + c), c);
  }
}

__global__ void __launch_bounds__(256)
quant_weight_kernel(const uint16_t* __restrict__ w, int8_t* __restrict__ q, float* __restrict__ scale,
                    int N, int K) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= N) return;
  const uint16_t* wp = w + (long)r * K;
  float amax = 0.f;
  for (int c = lane; c < K; c += 64) amax = fmaxf(amax, fabsf(bf2f(wp[c])));
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f);
  if (lane == 0) scale[r] = s;
  for (int c = lane; c < K; c += 64) {
    float v = rintf(__fdiv_rn(bf2f(wp[c]), s));
    v = fminf(fmaxf(v, -127.f), 127.f);
    q[(long)r * K + c] = (int8_t)(int)v;
  }
}

}  // namespace

hipError_t quant_rows_bf16(const uint16_t* x, long ldx, int8_t* q, long ldq, float* scale, int M, int K,
                           hipStream_t s, const int* M_dev) {
  if (M <= 0) return hipSuccess;
  if (K <= 0 || K % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0) return hipErrorInvalidValue;
  const dim3 grid((M + 3) / 4), block(256);
  switch (K) {
    case 1024:
      dfh_launch(quant_rows_kernel<2>, grid, block, 0, s, x, ldx, q, ldq, scale, M, K, M_dev);
      break;
    case 2048:
      dfh_launch(quant_rows_kernel<4>, grid, block, 0, s, x, ldx, q, ldq, scale, M, K, M_dev);
      break;
    case 4096:
      dfh_launch(quant_rows_kernel<8>, grid, block, 0, s, x, ldx, q, ldq, scale, M, K, M_dev);
      break;
    default:
      dfh_launch(quant_rows_kernel<0>, grid, block, 0, s, x, ldx, q, ldq, scale, M, K, M_dev);
      break;
  }
  return hipGetLastError();
}

hipError_t quant_weight_f32(const uint16_t* w, int8_t* q, float* scale, int N, int K, hipStream_t s) {
  if (N <= 0) return hipSuccess;
  if (K <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quant_weight_kernel, dim3((N + 3) / 4), dim3(256), 0, s, w, q, scale, N, K);
  return hipGetLastError();
}

}  // namespace dfh
