// int8 quantisation kernels of the W8A8 DiT linear (Int8DynamicLinear,
// nanovllm_dots/models/dots/int8_dit.py:34-65). HBM-bound, one wave per row.
//
// Activations (int8_dit.py:57-58) are quantised in the input dtype, bf16: every
// bf16 op is one IEEE float32 op rounded to nearest-even bf16, so
//   s = max(bf16(amax / 127), bf16(1e-8)),  q = clamp(rint(bf16(x / s)), -127, 127)
// with correctly rounded float32 division and round-half-to-even (v_rndne_f32).
// Weights (int8_dit.py:40-45) are quantised in float32:
//   s_w = max(amax / 127, 1e-8),  q = clamp(rint(w / s_w), -127, 127).
#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

__global__ void __launch_bounds__(256)
quant_rows_kernel(const uint16_t* __restrict__ x, long ldx, int8_t* __restrict__ q, long ldq,
                  float* __restrict__ scale, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= M) return;
  const uint16_t* xp = x + (long)r * ldx;
  float amax = 0.f;
  for (int c = lane * 8; c < K; c += 512) {
    const uint4 u = *reinterpret_cast<const uint4*>(xp + c);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      amax = fmaxf(amax, fabsf(bf2f((uint16_t)(w[t] & 0xffffu))));
      amax = fmaxf(amax, fabsf(bf2f((uint16_t)(w[t] >> 16))));
    }
  }
  amax = wave_max(amax);
  float s = rbf(__fdiv_rn(amax, 127.0f));
  s = fmaxf(s, rbf(1e-8f));
  if (lane == 0) scale[r] = s;
  int8_t* qp = q + (long)r * ldq;
  for (int c = lane * 8; c < K; c += 512) {
    const uint4 u = *reinterpret_cast<const uint4*>(xp + c);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint16_t h = (uint16_t)((t & 1) ? (w[t >> 1] >> 16) : (w[t >> 1] & 0xffffu));
      float v = rintf(rbf(__fdiv_rn(bf2f(h), s)));
      v = fminf(fmaxf(v, -127.f), 127.f);
      packed[t >> 2] |= ((uint32_t)(uint8_t)(int8_t)(int)v) << (8 * (t & 3));
    }
    *reinterpret_cast<uint2*>(qp + c) = make_uint2(packed[0], packed[1]);
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
                           hipStream_t s) {
  if (M <= 0) return hipSuccess;
  if (K <= 0 || K % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quant_rows_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, ldx, q, ldq, scale, M, K);
  return hipGetLastError();
}

hipError_t quant_weight_f32(const uint16_t* w, int8_t* q, float* scale, int N, int K, hipStream_t s) {
  if (N <= 0) return hipSuccess;
  if (K <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quant_weight_kernel, dim3((N + 3) / 4), dim3(256), 0, s, w, q, scale, N, K);
  return hipGetLastError();
}

}  // namespace dfh
