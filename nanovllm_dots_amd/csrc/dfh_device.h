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

// global / LDS address-space casts for __builtin_amdgcn_global_load_lds
#define DFH_GPTR(p) ((__attribute__((address_space(1))) void*)(p))
#define DFH_LPTR(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14])
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// s_waitcnt vmcnt(n) only (lgkmcnt and expcnt at their maxima: not waited for)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// float32 multiply / add that the compiler may not fuse into an FMA: sequences
// that reproduce torch's separately rounded elementwise ops use these.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));

// float -> bf16, round to nearest even (v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// two floats -> packed bf16 pair (low half = a), one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  floatx2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// round a float to the nearest bf16 value, returned as float
__device__ __forceinline__ float rbf(float f) { return (float)(__bf16)f; }

struct alignas(8) bf16q { bf16_t v[4]; };
struct alignas(16) bf16o { bf16_t v[8]; };

__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
  uint2 r;
  r.x = pack2(a, b);
  r.y = pack2(c, d);
  return r;
}

__device__ __forceinline__ void unpack4(uint2 r, float* o) {
  o[0] = bf2f((bf16_t)(r.x & 0xffffu));
  o[1] = bf2f((bf16_t)(r.x >> 16));
  o[2] = bf2f((bf16_t)(r.y & 0xffffu));
  o[3] = bf2f((bf16_t)(r.y >> 16));
}

// GELU, tanh approximation: 0.5*x*(1+tanh(u)), u = sqrt(2/pi)*(x+0.044715x^3), fp32.
// Evaluated as x * sigmoid(2u) = x / (1 + 2^(-2u*log2(e))): the same function
// (0.5*(1+tanh(u)) == sigmoid(2u)) with one exp2 and one reciprocal.
__device__ __forceinline__ float gelu_tanh_f(float x) {
  // -2*log2(e)*sqrt(2/pi) and its product with 0.044715
  const float c1 = -2.0f * 1.4426950408889634f * 0.7978845608028654f;
  const float c2 = c1 * 0.044715f;
  const float z = x * __builtin_fmaf(c2, x * x, c1);  // -2*log2(e)*u
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
// x * sigmoid(x) = x / (1 + 2^(-x*log2(e))) with one exp2 and one reciprocal
// (the GEMM epilogue's SiLU; within a few float32 ulp of silu_f)
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// value of lane l ^ 32 (the other half of the wave): one v_permlane32_swap,
// which exchanges lanes 32..63 of its first operand with lanes 0..31 of its
// second, instead of a ds_bpermute round trip through the LDS crossbar
__device__ __forceinline__ float swap_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

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
