// Device-side helpers shared by the FM/DiT head kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;  // raw bf16 bits in memory
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

#define DFH_WAVE 64

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// float -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ bf16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

// round a float to the nearest bf16 value, returned as float
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

struct alignas(8) bf16q { bf16_t v[4]; };
struct alignas(16) bf16o { bf16_t v[8]; };

__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
  uint2 r;
  r.x = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
  r.y = (uint32_t)f2bf(c) | ((uint32_t)f2bf(d) << 16);
  return r;
}

__device__ __forceinline__ void unpack4(uint2 r, float* o) {
  o[0] = bf2f((bf16_t)(r.x & 0xffffu));
  o[1] = bf2f((bf16_t)(r.x >> 16));
  o[2] = bf2f((bf16_t)(r.y & 0xffffu));
  o[3] = bf2f((bf16_t)(r.y >> 16));
}

// GELU, tanh approximation: 0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715x^3))), fp32.
__device__ __forceinline__ float gelu_tanh_f(float x) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  float x3 = x * x * x;
  float inner = k0 * (x + k1 * x3);
  return 0.5f * x * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// wave-wide reductions (64 lanes)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
