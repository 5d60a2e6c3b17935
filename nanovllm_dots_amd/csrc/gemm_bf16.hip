// bf16 GEMM on CDNA4 MFMA with fused DiT epilogues.
//
//   C[M, N] = A[M, K] * B[N, K]^T (+ bias)      (nn.Linear: y = x W^T + b)
//
// Both operands are K-contiguous, so every MFMA fragment is one 16-byte LDS
// read. The product is computed transposed (MFMA "A" operand = weight rows,
// "B" operand = activation rows): a lane of a 32x32 result block then owns one
// activation row m and runs of 4 consecutive output columns n, which gives
// 8-byte stores, register-local RoPE pairs (d, d+32) for the QKV epilogue and
// coalesced column writes of V^T.
//
// Schedule: persistent workgroups (grid = resident WGs), tiles walked in
// XCD-contiguous chunks so the row tiles that share A live in one XCD's L2.
// Operands move global -> LDS by DMA (global_load_lds_dwordx4: no staging
// registers, no ds_write) into ST statically distinct LDS stages: the DMA of K
// step k+ST-1 is issued while step k computes. Each step starts with an
// explicit wait for this wave's own DMA of step k (vmcnt) plus its LDS reads
// (lgkmcnt), then a barrier, so the step's tile is complete for every wave and
// the stage refilled next is no longer read by anyone.
#include <type_traits>

#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {


// K-loop schedules (per K step: wait for this wave's DMA of step k, barrier,
// DMA of step k+ST-1, fragment reads and MFMAs):
//  SCHED 0: every wave issues its share of the DMA.
//  SCHED 1: the DMA of step j is issued by one half of the workgroup (waves
//           4(j%2) .. 4(j%2)+3). The vector-memory path takes ~16 cycles per
//           1 KB DMA instruction, so a step's 64 instructions queue for ~1000
//           cycles and hold up the MFMAs of every wave that issued one; the half
//           that issues none starts its MFMAs right after the barrier.
//  SCHED 2: one wave per SIMD (4 waves, 128x128 per wave, accumulators in
//           AGPRs), BK 32 in 5 stages with the DMA 4 steps ahead. Each wave
//           spreads its DMA over its MFMAs, one 1 KB instruction after every 4
//           MFMAs: the vector-memory path (64 B per cycle per CU) absorbs the
//           CU's 4 instructions per 128 cycles as they come, so its queue never
//           fills and no wave stalls behind it. One barrier per step, between its
//           two 16-deep slices. The epilogue stages rows in the stage the next
//           tile's prologue leaves free. It needs a third fewer LDS fragment reads
//           per MFMA than SCHED 1; under random bf16 operands both run into the
//           chip's power limit at about the same rate, and SCHED 1 has the
//           smaller per-tile overhead, so production shapes use SCHED 1.
template <int BM_, int BN_, int BK_, int ST_, int WM_, int WN_, int SCHED_ = 0, int MAXSPLIT_ = 0,
          int MINSTEPS_ = 8>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, ST = ST_, WM = WM_, WN = WN_, SCHED = SCHED_;
  static constexpr int HD = SCHED == 1;  // the DMA of step j issued by half j % 2
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int NW = WM * WN;
  static constexpr int WTM = BM / WM;  // wave tile rows (activations)
  static constexpr int WTN = BN / WN;  // wave tile cols (outputs)
  static constexpr int RM = WTM / 32;
  static constexpr int RN = WTN / 32;
  static constexpr int CH = BK / 8;                 // 16-B chunks per LDS row
  static constexpr int ROWS_PER_DMA = 64 / CH;      // rows one wave fills per DMA (1 KB)
  static constexpr int DW = HD ? NW / 2 : NW;       // waves that issue one step's DMA
  static constexpr int RPR = DW * ROWS_PER_DMA;     // rows per DMA round of the workgroup
  static constexpr int AJ = BM / RPR, BJ = BN / RPR;
  static constexpr int LPS = AJ + BJ;               // DMA instructions per wave per K step
  // K pieces per leftover tile at most (its last piece reads the others' partial sums)
  static constexpr int MAX_SPLIT = MAXSPLIT_ ? MAXSPLIT_ : SCHED == 2 ? 2 : 64;
  // K steps per piece at least: the last piece's sum and epilogue cost per piece
  static constexpr int MIN_SPLIT_STEPS = MINSTEPS_;
  static constexpr int LDS_BYTES = ST * (BM + BN) * BK * 2;
  // two workgroups per CU when both fit in LDS (then <= 256 registers per lane)
  static constexpr int WG_PER_CU = (NW <= 4 && 2 * LDS_BYTES <= 160 * 1024) ? 2 : 1;
  static constexpr int WAVES_PER_EU = WG_PER_CU * NW / 4;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  static_assert(BM % RPR == 0 && BN % RPR == 0, "DMA rounds");
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(ST >= 1 && ST <= (SCHED == 2 ? 5 : 4), "stages");
  static_assert(!HD || NW == 8, "half DMA: 8 waves");
  static_assert(SCHED != 2 || (NW == 4 && ST == 5 && BK == 32 && AJ == 4 && BJ == 4 && RM * RN == 16),
                "SCHED 2: 4 waves, 128x128 per wave, BK 32 x 5 stages");
};

// LDS tile layout: rows of BK bf16 (BK/8 16-B chunks), row-major, logical chunk
// c of row r at slot c ^ swz(r). The LDS serves a ds_read_b128 sixteen lanes
// (256 B, 64 banks) at a time; a fragment read gives those lanes 16 consecutive
// rows at one logical chunk and the swizzle makes their 16-B bank groups
// (row, slot) -> (row*CH + slot) % 16 all distinct.
// buffer resource word 3 for gfx9-family raw (stride 0) buffers: 32-bit data format
constexpr int kBufferFlags = 0x00020000;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

template <int CH>
__device__ __forceinline__ int swz(int row) {
  return CH == 8 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}
template <int CH>
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * (CH * 8) + ((chunk ^ swz<CH>(row)) << 3);
}

// MFMA flavours sharing the tile machinery. An int8 row of K bytes has the byte
// layout of a bf16 row of K/2 elements, so the DMA / LDS / fragment code works
// on 16-bit units for both; one 16-byte fragment is 8 bf16 or 16 int8 values.
struct OpBf16 {
  using acc_t = floatx16;
  using elem_t = float;
  __device__ static __forceinline__ acc_t mma(const bf16x8& a, const bf16x8& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
struct OpI8 {
  using acc_t = intx16;
  using elem_t = int;
  __device__ static __forceinline__ acc_t mma(const bf16x8& a, const bf16x8& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(intx4, a), __builtin_bit_cast(intx4, b),
                                                  c, 0, 0, 0);
  }
};




// Epilogues whose bf16 output goes through LDS: each wave writes one 32-row
// block of its tile into a private region of the stage the main loop is not
// filling, then stores it back as whole rows, 16 B per lane (8 full 128-B rows
// per store instruction instead of 32 partial rows). Needs NW * 32 * WTN bf16
// of free stage: half the waves in the A buffer, half in the B buffer.
// The gate-residual epilogue reads its residual and gate rows the same way,
// 16 B per lane, one 32-row block ahead of the block it stores.
template <class C, int EPI>
struct Staged {
  static constexpr int B = base_epi(EPI);
  static constexpr bool kEpi = B == EPI_BIAS || B == EPI_GELU || B == EPI_SILU || B == EPI_GATE_RES;
  static constexpr int kSmall = C::BM < C::BN ? C::BM : C::BN;
  static constexpr bool value = kEpi && (C::NW / 2) * 32 * C::WTN <= kSmall * C::BK && C::NW % 2 == 0;
  static constexpr int CPR = C::WTN / 8;   // 16-B chunks per staged row
  static constexpr int RPI = 64 / CPR;     // rows per wave-wide 16-B access
  static constexpr int JB = 32 / RPI;      // wave-wide accesses per 32-row block
  static constexpr int kStores = C::RM * JB;
  static constexpr bool kRes = B == EPI_GATE_RES;
  // vector-memory ops the epilogue issues after the next tile's prologue DMA
  // (stores, and the residual + gate loads of blocks 1 .. RM-1), on every path
  static constexpr int kVmAfter = kStores + (kRes ? (C::RM - 1) * 2 * JB : 0);
};

// staged element offset: row r (0..31) of the block, 16-B chunk c, slot c ^ ((r >> 1) & 7)
template <int CPR>
__device__ __forceinline__ int stage_off(int r, int c) {
  return r * CPR * 8 + ((c ^ ((r >> 1) & (CPR - 1))) << 3);
}

// Column operands of a staged epilogue (bias, int8 weight scales) and the row
// scales of W8A8, loaded BEFORE the next tile's prologue DMA: vmcnt completes
// in issue order, so a later load would make its first use wait for that DMA.
template <class C, int EPI>
struct StagedOperands {
  static constexpr int JB = Staged<C, EPI>::JB, NRES = Staged<C, EPI>::kRes ? JB : 1;
  float b[C::RN][4][4];
  float w[is_dq(EPI) ? C::RN : 1][4][4];
  float sx[is_dq(EPI) ? C::RM : 1];
  uint4 x0[NRES], g0[NRES];  // gate-residual: residual and gate chunks of block 0
};

// Gate-residual rows a lane stores: row j*RPI + lane/CPR of each 32-row block,
// columns (lane % CPR)*8 .. +8. Their requests (row -> request table) are read
// at the start of the tile, so the gate address is known when the epilogue needs it.
template <class C, int EPI>
struct ResRows {
  int rq[Staged<C, EPI>::kRes ? C::RM * Staged<C, EPI>::JB : 1];
};
template <class C, int EPI>
__device__ __forceinline__ void res_rows_load(const GemmArgs& a, ResRows<C, EPI>& rr, int m0, int M, int wm,
                                              int lane) {
  if constexpr (Staged<C, EPI>::kRes && Staged<C, EPI>::value) {
    using S = Staged<C, EPI>;
#pragma unroll
    for (int k = 0; k < C::RM; ++k)
#pragma unroll
      for (int j = 0; j < S::JB; ++j) {
        const int m = m0 + wm * C::WTM + k * 32 + j * S::RPI + lane / S::CPR;
        rr.rq[k * S::JB + j] = a.row_req[m < M ? m : M - 1];
      }
  }
}
// residual and gate chunks of block k (rows clamped to M - 1: always issued)
template <class C, int EPI>
__device__ __forceinline__ void res_block_load(const GemmArgs& a, const ResRows<C, EPI>& rr, int k, int m0, int n0,
                                               int M, int wm, int wn, int lane, uint4 (&x)[Staged<C, EPI>::JB],
                                               uint4 (&g)[Staged<C, EPI>::JB]) {
  using S = Staged<C, EPI>;
  const int n = n0 + wn * C::WTN + (lane % S::CPR) * 8;
#pragma unroll
  for (int j = 0; j < S::JB; ++j) {
    const int m = m0 + wm * C::WTM + k * 32 + j * S::RPI + lane / S::CPR;
    const int mm = m < M ? m : M - 1;
    x[j] = *reinterpret_cast<const uint4*>(a.res ? a.res + (long)mm * a.ld_res + n : a.C + (long)mm * a.ldc + n);
    g[j] = *reinterpret_cast<const uint4*>(a.gate + (long)rr.rq[k * S::JB + j] * a.ld_gate + n);
  }
}

template <class C, int EPI>
__device__ __forceinline__ void staged_preload(const GemmArgs& a, StagedOperands<C, EPI>& op,
                                               const ResRows<C, EPI>& rr, int m0, int n0, int M, int wm, int wn,
                                               int lane, int l32, int hi) {
  // one uniform branch around all loads, so they issue back to back and are waited for once
  uint2 braw[C::RN][4];
  if (a.bias) {
#pragma unroll
    for (int i = 0; i < C::RN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        braw[i][g] = *reinterpret_cast<const uint2*>(a.bias + n0 + wn * C::WTN + i * 32 + 8 * g + 4 * hi);
  } else {
#pragma unroll
    for (int i = 0; i < C::RN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) braw[i][g] = make_uint2(0u, 0u);
  }
#pragma unroll
  for (int i = 0; i < C::RN; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + wn * C::WTN + i * 32 + 8 * g + 4 * hi;
      unpack4(braw[i][g], op.b[i][g]);
      if constexpr (is_dq(EPI)) {
        const float4 w4 = *reinterpret_cast<const float4*>(a.sw + n);
        op.w[i][g][0] = w4.x; op.w[i][g][1] = w4.y; op.w[i][g][2] = w4.z; op.w[i][g][3] = w4.w;
      }
    }
  if constexpr (is_dq(EPI)) {
#pragma unroll
    for (int k = 0; k < C::RM; ++k) {
      const int m = m0 + wm * C::WTM + k * 32 + l32;
      op.sx[k] = a.sx[m < M ? m : M - 1];
    }
  }
  if constexpr (Staged<C, EPI>::kRes) res_block_load<C, EPI>(a, rr, 0, m0, n0, M, wm, wn, lane, op.x0, op.g0);
}

template <class C, int EPI, class ACC>
__device__ __forceinline__ void staged_epilogue(const GemmArgs& a, ACC (&acc)[C::RN][C::RM],
                                                const StagedOperands<C, EPI>& op, const ResRows<C, EPI>& rr,
                                                int m0, int n0, int M, int wm, int wn, int lane, int l32, int hi,
                                                uint16_t* region) {
  using S = Staged<C, EPI>;
  constexpr int CPR = S::CPR, RPI = S::RPI, JB = S::JB, NB = S::kRes ? 2 : 1, NJ = S::kRes ? JB : 1;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.C + (long)m0 * a.ldc), (short)0, (int)((uint32_t)(M - m0) * (uint32_t)a.ldc * 2u), kBufferFlags);
  const int ncol0 = n0 + wn * C::WTN;
  // gate-residual: residual / gate chunks, double-buffered by block
  uint4 xb[NB][NJ], gb[NB][NJ];
  if constexpr (S::kRes) {
#pragma unroll
    for (int j = 0; j < JB; ++j) { xb[0][j] = op.x0[j]; gb[0][j] = op.g0[j]; }
  }
#pragma unroll
  for (int k = 0; k < C::RM; ++k) {
    // MFMA layout -> LDS: lane (l32, hi) holds row l32, columns i*32 + 8g + 4hi + [0, 4)
#pragma unroll
    for (int i = 0; i < C::RN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float y[4];
        if constexpr (is_dq(EPI)) {
          // ((acc.f32 * s_x) * s_w) + bias, each op rounded to float32 (int8_dit.py:60-62)
#pragma unroll
          for (int t = 0; t < 4; ++t)
            y[t] = add_rn(mul_rn(mul_rn((float)acc[i][k][4 * g + t], op.sx[k]), op.w[i][g][t]), op.b[i][g][t]);
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) y[t] = acc[i][k][4 * g + t] + op.b[i][g][t];
        }
        if constexpr (base_epi(EPI) == EPI_GELU) {
#pragma unroll
          for (int t = 0; t < 4; ++t) y[t] = gelu_tanh_f(rbf(y[t]));
        } else if constexpr (base_epi(EPI) == EPI_SILU) {
#pragma unroll
          for (int t = 0; t < 4; ++t) y[t] = silu_fast(rbf(y[t]));
        }
        *reinterpret_cast<uint2*>(region + stage_off<CPR>(l32, 4 * i + g) + 4 * hi) = pack4(y[0], y[1], y[2], y[3]);
      }
    // the next block's residual / gate reads go out before this block's stores,
    // so waiting for them later never waits for these stores
    if constexpr (S::kRes) {
      if (k + 1 < C::RM) res_block_load<C, EPI>(a, rr, k + 1, m0, n0, M, wm, wn, lane, xb[(k + 1) & 1], gb[(k + 1) & 1]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // LDS -> rows: lane reads 16 B of row j*RPI + lane/CPR and stores it
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int r = j * RPI + lane / CPR, c = lane % CPR;
      uint4 v = *reinterpret_cast<const uint4*>(region + stage_off<CPR>(r, c));
      if constexpr (S::kRes) {
        // out = x + bf16(gate * bf16(y)), y = acc + bias already rounded to bf16 in LDS
        float yv[8], xv[8], gv[8];
        unpack4(make_uint2(v.x, v.y), yv);
        unpack4(make_uint2(v.z, v.w), yv + 4);
        const uint4 xq = xb[k & 1][j], gq = gb[k & 1][j];
        unpack4(make_uint2(xq.x, xq.y), xv);
        unpack4(make_uint2(xq.z, xq.w), xv + 4);
        unpack4(make_uint2(gq.x, gq.y), gv);
        unpack4(make_uint2(gq.z, gq.w), gv + 4);
        float o[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t] = xv[t] + rbf(gv[t] * yv[t]);
        const uint2 lo = pack4(o[0], o[1], o[2], o[3]), hi2 = pack4(o[4], o[5], o[6], o[7]);
        v = make_uint4(lo.x, lo.y, hi2.x, hi2.y);
      }
      const int rt = wm * C::WTM + k * 32 + r;  // row within the tile
      const int n = ncol0 + c * 8;
      const u32x4 o = {v.x, v.y, v.z, v.w};
      __builtin_amdgcn_raw_buffer_store_b128(o, rc, ((uint32_t)rt * (uint32_t)a.ldc + (uint32_t)n) * 2u, 0, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next block overwrites
  }
}

// q / k: bias, optional per-head LayerNorm / RMSNorm over 64, RoPE on the
// column pairs (d, d+32) that a lane holds in blocks (i, i+1); v: transposed
// into V^T[column][vt_col[row]].
template <class C, bool DQ, class ACC>
__device__ __forceinline__ void qkv_epilogue(const GemmArgs& a, ACC (&acc)[C::RN][C::RM], int m0, int n0,
                                             int M, int wm, int wn, int l32, int hi) {
  const int H = a.hidden;
  // the linear's output of accumulator e, output column n (within q|k|v), bias b:
  // acc + b, or with int8 operands ((acc * s_x) * s_w) + b (int8_dit.py:60-62)
  auto lin = [&](auto e, float sxm, int n, float b) {
    if constexpr (DQ) return add_rn(mul_rn(mul_rn((float)e, sxm), a.sw[n]), b);
    else return (float)e + b;
  };
  n0 += a.col0;               // column within the fused q|k|v output
  const int region = n0 / H;  // 0 q, 1 k, 2 v (BN divides H)
#pragma unroll
  for (int k = 0; k < C::RM; ++k) {
    const int m = m0 + wm * C::WTM + k * 32 + l32;
    const bool valid = m < M;
    const int mm = valid ? m : M - 1;
    const float sxm = DQ ? a.sx[mm] : 0.f;
    if (region == 2) {
      const int col = a.vt_col[mm];
#pragma unroll
      for (int i = 0; i < C::RN; ++i) {
        const int nb = n0 + wn * C::WTN + i * 32 - 2 * H;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int n = nb + 8 * (v >> 2) + 4 * hi + (v & 3);
          float y = lin(acc[i][k][v], sxm, n + 2 * H, a.bias ? bf2f(a.bias[n + 2 * H]) : 0.f);
          if (valid) a.vt[(long)n * a.ld_vt + col] = f2bf(y);
        }
      }
      continue;
    }
    const uint16_t* nw = region == 0 ? a.qn_w : a.kn_w;
    const uint16_t* nbias = region == 0 ? a.qn_b : a.kn_b;
    const int pos = a.row_pos[mm];
    // heads are pairs of 32-column blocks (i, i+1): d in [0,32) and [32,64)
#pragma unroll
    for (int i = 0; i < C::RN; i += 2) {
      const int nb = n0 + wn * C::WTN + i * 32;  // head start column (within q|k|v)
      float x0[16], x1[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int d = 8 * (v >> 2) + 4 * hi + (v & 3);
        float b0 = a.bias ? bf2f(a.bias[nb + d]) : 0.f;
        float b1 = a.bias ? bf2f(a.bias[nb + 32 + d]) : 0.f;
        x0[v] = rbf(lin(acc[i][k][v], sxm, nb + d, b0));
        x1[v] = rbf(lin(acc[i + 1][k][v], sxm, nb + 32 + d, b1));
      }
      if (a.qk_norm) {
        float s = 0.f, s2 = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) { s += x0[v] + x1[v]; }
        s += __shfl_xor(s, 32, 64);
        float mean = a.qk_norm == 1 ? s * (1.0f / 64.0f) : 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float d0 = x0[v] - mean, d1 = x1[v] - mean;
          s2 += d0 * d0 + d1 * d1;
        }
        s2 += __shfl_xor(s2, 32, 64);
        const float eps = a.qk_norm == 1 ? 1e-5f : 1.1920928955078125e-07f;
        const float rstd = rsqrtf(s2 * (1.0f / 64.0f) + eps);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int d = 8 * (v >> 2) + 4 * hi + (v & 3);
          float w0 = bf2f(nw[d]), w1 = bf2f(nw[d + 32]);
          float c0 = (a.qk_norm == 1) ? bf2f(nbias[d]) : 0.f;
          float c1 = (a.qk_norm == 1) ? bf2f(nbias[d + 32]) : 0.f;
          x0[v] = (x0[v] - mean) * rstd * w0 + c0;
          x1[v] = (x1[v] - mean) * rstd * w1 + c1;
        }
      }
      if (a.rope_cos && !(region == 0 && a.rope_q_in_attn)) {
        // tables grouped by 32 positions (rope_table): this lane's d = 8g + 4hi + t
        const long to = ((long)(pos >> 5) * 256 + (pos & 31) * 2 + hi) * 4;
        const float* cs = a.rope_cos + to;
        const float* sn = a.rope_sin + to;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int tg = (v >> 2) * 256 + (v & 3);
          const float c = cs[tg], s = sn[tg];
          const float r0 = add_rn(mul_rn(x0[v], c), mul_rn(-x1[v], s));
          const float r1 = add_rn(mul_rn(x1[v], c), mul_rn(x0[v], s));
          x0[v] = r0;
          x1[v] = r1;
        }
      }
      if (valid) {
        uint16_t* cp = a.C + (long)(a.c_rows ? a.c_rows[m] : m) * a.ldc + nb;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 8 * g + 4 * hi;
          *reinterpret_cast<uint2*>(cp + d) = pack4(x0[4 * g], x0[4 * g + 1], x0[4 * g + 2], x0[4 * g + 3]);
          *reinterpret_cast<uint2*>(cp + 32 + d) = pack4(x1[4 * g], x1[4 * g + 1], x1[4 * g + 2], x1[4 * g + 3]);
        }
      }
    }
  }
}

// QKV epilogue with a fixed number of stores per lane (bf16 operands; no
// qk-norm, no output-row table). Every load comes before the first store: the
// row tables of all row blocks and the bias at the start, block k+1's RoPE
// factors before block k's stores, so no load waits for a store. The stores
// go through buffer resources that drop rows at or past M instead of a row
// branch, so a lane issues RM * RN * 4 of them on a q|k tile and
// RM * RN * 16 on a V tile, and the next tile's first K step waits for its
// prologue DMA only. Same values as qkv_epilogue. Returns 0 (q|k tile),
// 1 (V tile) or 2 (qkv_epilogue ran: the next step waits for everything).
template <class C>
__device__ __forceinline__ int qkv_epilogue_fixed(const GemmArgs& a, floatx16 (&acc)[C::RN][C::RM], int m0,
                                                  int n0, int M, int wm, int wn, int l32, int hi) {
  const int H = a.hidden;
  if (a.qk_norm || a.c_rows || (long)H * a.ld_vt * 2 >= 0x7fffffffL) {  // uniform
    qkv_epilogue<C, false>(a, acc, m0, n0, M, wm, wn, l32, hi);
    return 2;
  }
  const int nq = n0 + a.col0 + wn * C::WTN;  // this wave's first column within q|k|v (= column of C)
  const int region = (n0 + a.col0) / H;      // 0 q, 1 k, 2 v (BN divides H)
  int rt[C::RM];                             // per row block: V^T column (v) or position (q, k)
#pragma unroll
  for (int k = 0; k < C::RM; ++k) {
    const int m = m0 + wm * C::WTM + k * 32 + l32;
    const int mm = m < M ? m : M - 1;
    rt[k] = region == 2 ? a.vt_col[mm] : a.row_pos[mm];
  }
  // bias of this lane's columns i*32 + 8g + 4hi + [0, 4)
  uint2 braw[C::RN][4];
#pragma unroll
  for (int i = 0; i < C::RN; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      braw[i][g] = a.bias ? *reinterpret_cast<const uint2*>(a.bias + nq + i * 32 + 8 * g + 4 * hi)
                          : make_uint2(0u, 0u);
  auto bias = [&](int i, int v) {
    const uint32_t w = (v & 2) ? braw[i][v >> 2].y : braw[i][v >> 2].x;
    return bf2f((bf16_t)((v & 1) ? w >> 16 : w & 0xffffu));
  };
  if (region == 2) {
    // V^T[n][vt_col[m]], 2 B per store; rows at or past M get an offset past the range
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.vt, (short)0, 0x7fffffff, kBufferFlags);
#pragma unroll
    for (int k = 0; k < C::RM; ++k) {
      const bool valid = m0 + wm * C::WTM + k * 32 + l32 < M;
#pragma unroll
      for (int i = 0; i < C::RN; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t n = (uint32_t)(nq - 2 * H + i * 32 + 8 * (v >> 2) + 4 * hi + (v & 3));
          const float y = (float)acc[i][k][v] + bias(i, v);
          const uint32_t off = valid ? (n * (uint32_t)a.ld_vt + (uint32_t)rt[k]) * 2u : 0xffffffffu;
          __builtin_amdgcn_raw_buffer_store_b16(f2bf(y), rv, off, 0, 0);
        }
    }
    return 1;
  }
  // q / k rows of this tile: rows at or past M fall outside the range
  const int rows = M - m0 < C::BM ? M - m0 : C::BM;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.C + (long)m0 * a.ldc), (short)0, (int)((uint32_t)rows * (uint32_t)a.ldc * 2u), kBufferFlags);
  const bool rope = a.rope_cos && !(region == 0 && a.rope_q_in_attn);  // uniform
  // RoPE factors of one row block: tables grouped by 32 positions (rope_table),
  // this lane's d = 8g + 4hi + t
  float4 cf[4], sf[4];
  auto rope_load = [&](int pos) {
    const long to = ((long)(pos >> 5) * 256 + (pos & 31) * 2 + hi) * 4;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      cf[g] = *reinterpret_cast<const float4*>(a.rope_cos + to + g * 256);
      sf[g] = *reinterpret_cast<const float4*>(a.rope_sin + to + g * 256);
    }
  };
  if (rope) rope_load(rt[0]);
#pragma unroll
  for (int k = 0; k < C::RM; ++k) {
    const uint32_t rowoff = (uint32_t)(wm * C::WTM + k * 32 + l32) * (uint32_t)a.ldc;
    uint2 out[C::RN >= 2 ? C::RN / 2 : 1][8];
    // heads are pairs of 32-column blocks (i, i+1): d in [0,32) and [32,64)
#pragma unroll
    for (int i = 0; i < C::RN; i += 2) {
      float x0[16], x1[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        x0[v] = rbf((float)acc[i][k][v] + bias(i, v));
        x1[v] = rbf((float)acc[i + 1][k][v] + bias(i + 1, v));
      }
      if (rope) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float4 c4 = cf[v >> 2], s4 = sf[v >> 2];
          const int t = v & 3;
          const float c = t == 0 ? c4.x : t == 1 ? c4.y : t == 2 ? c4.z : c4.w;
          const float sn = t == 0 ? s4.x : t == 1 ? s4.y : t == 2 ? s4.z : s4.w;
          const float r0 = add_rn(mul_rn(x0[v], c), mul_rn(-x1[v], sn));
          const float r1 = add_rn(mul_rn(x1[v], c), mul_rn(x0[v], sn));
          x0[v] = r0;
          x1[v] = r1;
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        out[i / 2][g] = pack4(x0[4 * g], x0[4 * g + 1], x0[4 * g + 2], x0[4 * g + 3]);
        out[i / 2][4 + g] = pack4(x1[4 * g], x1[4 * g + 1], x1[4 * g + 2], x1[4 * g + 3]);
      }
    }
    // the next block's factors go out before this block's stores
    if (rope && k + 1 < C::RM) rope_load(rt[k + 1]);
#pragma unroll
    for (int i = 0; i < C::RN; i += 2)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t col = (uint32_t)(nq + i * 32 + 8 * g + 4 * hi);
        const u32x2 lo = {out[i / 2][g].x, out[i / 2][g].y}, hi2 = {out[i / 2][4 + g].x, out[i / 2][4 + g].y};
        __builtin_amdgcn_raw_buffer_store_b64(lo, rc, (rowoff + col) * 2u, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(hi2, rc, (rowoff + col + 32u) * 2u, 0, 0);
      }
  }
  return 0;
}

template <class C, int EPI, class ACC>
__device__ __forceinline__ void run_epilogue(const GemmArgs& a, ACC (&acc)[C::RN][C::RM], int m0,
                                             int n0, int M, int wm, int wn, int l32, int hi) {
    if constexpr (base_epi(EPI) == EPI_QKV) {
      qkv_epilogue<C, is_dq(EPI)>(a, acc, m0, n0, M, wm, wn, l32, hi);
    } else {
      // bias (and int8 weight scale) of this lane's output columns, hoisted out of
      // the row loop for narrow wave tiles (wide ones reload them: registers)
      constexpr bool kHoist = C::RN <= 2;
      constexpr int HN = kHoist ? C::RN : 1;
      float bv[HN][4][4];
      float swv[HN][4][4];
      auto load_cols = [&](int i, int hi_, float (&b4)[4][4], float (&w4)[4][4]) {
        uint2 braw[4];
        if (a.bias) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
            braw[g] = *reinterpret_cast<const uint2*>(a.bias + n0 + wn * C::WTN + i * 32 + 8 * g + 4 * hi_);
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) braw[g] = make_uint2(0u, 0u);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * C::WTN + i * 32 + 8 * g + 4 * hi_;
          unpack4(braw[g], b4[g]);
          if constexpr (is_dq(EPI)) {
            const float4 q4 = *reinterpret_cast<const float4*>(a.sw + n);
            w4[g][0] = q4.x; w4[g][1] = q4.y; w4[g][2] = q4.z; w4[g][3] = q4.w;
          }
        }
      };
      if constexpr (kHoist) {
#pragma unroll
        for (int i = 0; i < C::RN; ++i) load_cols(i, hi, bv[i], swv[i]);
      }
      // Rows [m0, M) of the output through a range-limited buffer resource:
      // stores to rows at or past M are dropped by the hardware, so the
      // epilogue has no row branches and always issues RN*RM*4 stores (the
      // tile-start wait of the main loop counts on that). Table lookups and
      // residual reads use the row clamped to M - 1.
      constexpr int ESZ = (EPI == EPI_F32 || EPI == EPI_I32) ? 4 : 2;
      void* cbase = EPI == EPI_F32 ? (void*)(a.Cf + (long)m0 * a.ldc)
                  : EPI == EPI_I32 ? (void*)(a.Ci + (long)m0 * a.ldc)
                                   : (void*)(a.C + (long)m0 * a.ldc);
      const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
          cbase, (short)0, (int)((uint32_t)(M - m0) * (uint32_t)a.ldc * (uint32_t)ESZ), kBufferFlags);
#pragma unroll
      for (int k = 0; k < C::RM; ++k) {
        const int r = wm * C::WTM + k * 32 + l32;  // row within the tile
        const int mm = m0 + r < M ? m0 + r : M - 1;
        const uint32_t rowoff = (uint32_t)r * (uint32_t)a.ldc;
        const uint16_t* xrow = a.res ? a.res + (long)mm * a.ld_res : a.C + (long)mm * a.ldc;
        const uint16_t* grow = nullptr;
        if constexpr (base_epi(EPI) == EPI_GATE_RES) grow = a.gate + (long)a.row_req[mm] * a.ld_gate;
        float sxm = 0.f;
        if constexpr (is_dq(EPI)) sxm = a.sx[mm];
#pragma unroll
        for (int i = 0; i < C::RN; ++i) {
          const int nb = n0 + wn * C::WTN + i * 32 + 4 * hi;
          float (&bvi)[4][4] = bv[kHoist ? i : 0];
          float (&swi)[4][4] = swv[kHoist ? i : 0];
          if constexpr (!kHoist) load_cols(i, hi, bvi, swi);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int n = nb + 8 * g;
            const uint32_t off = (rowoff + (uint32_t)n) * (uint32_t)ESZ;
            float y[4];
            if constexpr (EPI == EPI_I32) {
              const u32x4 v = {(uint32_t)acc[i][k][4 * g], (uint32_t)acc[i][k][4 * g + 1],
                               (uint32_t)acc[i][k][4 * g + 2], (uint32_t)acc[i][k][4 * g + 3]};
              __builtin_amdgcn_raw_buffer_store_b128(v, rc, off, 0, 0);
              continue;
            } else if constexpr (is_dq(EPI)) {
              // ((acc.f32 * s_x) * s_w) + bias, each op rounded to float32 (int8_dit.py:60-62)
#pragma unroll
              for (int t = 0; t < 4; ++t)
                y[t] = add_rn(mul_rn(mul_rn((float)acc[i][k][4 * g + t], sxm), swi[g][t]), bvi[g][t]);
            } else {
#pragma unroll
              for (int t = 0; t < 4; ++t) y[t] = acc[i][k][4 * g + t] + bvi[g][t];
            }
            if constexpr (EPI == EPI_F32) {
              const u32x4 v = {__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                               __float_as_uint(y[3])};
              __builtin_amdgcn_raw_buffer_store_b128(v, rc, off, 0, 0);
              continue;
            } else if constexpr (base_epi(EPI) == EPI_GELU) {
#pragma unroll
              for (int t = 0; t < 4; ++t) y[t] = gelu_tanh_f(rbf(y[t]));
            } else if constexpr (base_epi(EPI) == EPI_SILU) {
#pragma unroll
              for (int t = 0; t < 4; ++t) y[t] = silu_fast(rbf(y[t]));
            } else if constexpr (base_epi(EPI) == EPI_GATE_RES) {
              float gt[4], xr[4];
              unpack4(*reinterpret_cast<const uint2*>(grow + n), gt);
              unpack4(*reinterpret_cast<const uint2*>(xrow + n), xr);
#pragma unroll
              for (int t = 0; t < 4; ++t) y[t] = xr[t] + rbf(gt[t] * rbf(y[t]));
            }
            // EPI_BIAS: one rounding, inside the pack
            const uint2 pk = pack4(y[0], y[1], y[2], y[3]);
            const u32x2 v = {pk.x, pk.y};
            __builtin_amdgcn_raw_buffer_store_b64(v, rc, off, 0, 0);
          }
        }
      }
    }
}

// K-split of an XCD's last round: chunk_x tiles over per_xcd workgroups leave
// tail = chunk_x mod per_xcd tiles for a partial round. Cut each of them into
// split = per_xcd / tail K pieces (at least min_steps K steps each) so the
// round takes 1/split of a tile instead of a whole one.
// workspace layout: kSplitCounters 32-bit tile counters (index xcd * per_xcd +
// leftover tile; at a fixed place for every tile shape, zero between calls),
// then one BM x BN float32 partial tile per workgroup
constexpr long kSplitCounters = 4096;
__device__ __forceinline__ void split_plan(int chunk_x, int per_xcd, int KT, int max_split, int min_steps,
                                           int& full_x, int& split) {
  full_x = chunk_x;
  split = 1;
  const int rounds = chunk_x / per_xcd, tail = chunk_x - rounds * per_xcd;
  if (tail == 0) return;
  int sp = per_xcd / tail;
  if (sp > KT / min_steps) sp = KT / min_steps;
  if (sp > max_split) sp = max_split;
  if (sp < 2) return;
  full_x = rounds * per_xcd;
  split = sp;
}

template <class C, class Op, int EPI>
__global__ void __launch_bounds__(C::THREADS, C::WAVES_PER_EU)
gemm_mfma_kernel(GemmArgs a) {
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, ST = C::ST, CH = C::CH, TH = C::THREADS;
  // one distinct LDS object per stage: the compiler can then prove that the DMA
  // into one stage never aliases LDS reads of another, and inserts no wait for it
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[BM * BK], sB0[BN * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[ST > 1 ? BM * BK : 8], sB1[ST > 1 ? BN * BK : 8];
  __shared__ __attribute__((aligned(1024))) uint16_t sA2[ST > 2 ? BM * BK : 8], sB2[ST > 2 ? BN * BK : 8];
  __shared__ __attribute__((aligned(1024))) uint16_t sA3[ST > 3 ? BM * BK : 8], sB3[ST > 3 ? BN * BK : 8];
  __shared__ __attribute__((aligned(1024))) uint16_t sA4[ST > 4 ? BM * BK : 8], sB4[ST > 4 ? BN * BK : 8];
  // K-split: this workgroup completed its tile. Kept in stage 0, which no DMA
  // fills and no epilogue stages into while the flag is in use.
  int& s_flag = *reinterpret_cast<int*>(sA0);
  auto stA = [&](auto stc) -> uint16_t* {
    constexpr int s = decltype(stc)::value;
    if constexpr (s == 0) return sA0;
    else if constexpr (s == 1) return sA1;
    else if constexpr (s == 2) return sA2;
    else if constexpr (s == 3) return sA3;
    else return sA4;
  };
  auto stB = [&](auto stc) -> uint16_t* {
    constexpr int s = decltype(stc)::value;
    if constexpr (s == 0) return sB0;
    else if constexpr (s == 1) return sB1;
    else if constexpr (s == 2) return sB2;
    else if constexpr (s == 3) return sB3;
    else return sB4;
  };

  const int M = a.M_dev ? *a.M_dev : a.M;
  const int N = a.N, K = a.K;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  if (total == 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS / DMA bases in SGPRs
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int l32 = lane & 31, hi = lane >> 5;

  // XCD-contiguous tile walk: workgroups with equal blockIdx.x % 8 share an XCD.
  const int nxcd = 8;
  const int xcd = blockIdx.x % nxcd;
  const int slot = blockIdx.x / nxcd;
  const int per_xcd = gridDim.x / nxcd;
  const int chunk = (total + nxcd - 1) / nxcd;
  // Work of this workgroup: whole tiles jt = slot, slot + per_xcd, ... < full_x
  // of the XCD's chunk, then (split > 1) one K piece of a leftover tile.
  int chunk_x = total - xcd * chunk;
  chunk_x = chunk_x < 0 ? 0 : (chunk_x > chunk ? chunk : chunk_x);
  int full_x = chunk_x, split = 1;
  if (a.ws != nullptr) split_plan(chunk_x, per_xcd, K / BK, C::MAX_SPLIT, C::MIN_SPLIT_STEPS, full_x, split);
  auto tile_at = [&](int jt) { return jt < full_x ? xcd * chunk + jt : -1; };
  // Grouped order: the per_xcd tiles an XCD runs at once cover GM row blocks x
  // per_xcd/GM column blocks (row block fastest), so each A row block and W
  // column block is fetched into that XCD's L2 once per round, not per tile.
  // Four column blocks per round (eight row blocks of 256 rows, sixteen of
  // 128): measured, fc1 0.5-2 % and the O projection 2-5 % faster than eight,
  // and the K|V-only projection (eight column blocks) 4 % faster. The full
  // q|k|v projection (twelve) runs 0.5-1 % faster with eight.
  const int gn_max = base_epi(EPI) == EPI_QKV && tiles_n > 8 ? 8 : 4;
  const int gn = tiles_n < gn_max ? tiles_n : gn_max;
  const int GM = per_xcd / gn > 1 ? per_xcd / gn : 1;
  auto tile_mn = [&](int t, int& m0, int& n0) {
    const int gsz = GM * tiles_n;
    const int g = t / gsz, w = t - g * gsz;
    const int gm0 = g * GM;
    const int rows = tiles_m - gm0 < GM ? tiles_m - gm0 : GM;
    m0 = (gm0 + w % rows) * BM;
    n0 = (w / rows) * BN;
  };

  // DMA: lane L of wave w, load j -> tile row j*RPR + w*ROWS_PER_DMA + L/CH, slot L%CH,
  // i.e. source chunk (L%CH) ^ swz(row); swz(row) is the same for every j (RPR % 16 == 0).
  // Buffer loads with a per-tile resource: rows at or past M fall outside the
  // resource's range and arrive as zeros, so no row clamping; per lane only one
  // 32-bit byte offset per operand stays live.
  static_assert(C::RPR % 16 == 0, "swizzle must not depend on the DMA round");
  const int dma_wave = wave % C::DW;
  const int dma_row = dma_wave * C::ROWS_PER_DMA + lane / CH;
  const uint32_t dma_col = (uint32_t)(((lane % CH) ^ swz<CH>(dma_row)) << 3);
  const uint32_t va = ((uint32_t)dma_row * (uint32_t)a.lda + dma_col) * 2u;
  const uint32_t vb = ((uint32_t)dma_row * (uint32_t)a.ldb + dma_col) * 2u;
  const uint32_t a_round = (uint32_t)C::RPR * (uint32_t)a.lda * 2u;
  const uint32_t b_round = (uint32_t)C::RPR * (uint32_t)a.ldb * 2u;
  __amdgpu_buffer_rsrc_t ra, rb;
  auto set_offsets = [&](int tile) {
    int m0, n0;
    tile_mn(tile, m0, n0);
    ra = __builtin_amdgcn_make_buffer_rsrc((void*)(a.A + (long)m0 * a.lda), (short)0,
                                           (int)((uint32_t)(M - m0) * (uint32_t)a.lda * 2u), kBufferFlags);
    rb = __builtin_amdgcn_make_buffer_rsrc((void*)(a.B + (long)n0 * a.ldb), (short)0,
                                           (int)((uint32_t)BN * (uint32_t)a.ldb * 2u), kBufferFlags);
  };
  auto dma = [&](auto stc, int kstep) {
    if (C::HD && (wave >> 2) != (kstep & 1)) return;  // uniform per wave
    uint16_t* la = stA(stc);
    uint16_t* lb = stB(stc);
    const int koff = kstep * BK * 2;
    // the per-round offsets are recomputed here (the empty asm hides them from
    // loop-invariant hoisting, which would pin AJ + BJ registers for the whole kernel)
    uint32_t vo = va;
#pragma unroll
    for (int j = 0; j < C::AJ; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, DFH_LPTR(la + (j * C::RPR + dma_wave * C::ROWS_PER_DMA) * BK),
                                               16, vo, koff, 0, 0);
      vo += a_round;
      asm volatile("" : "+v"(vo));
    }
    vo = vb;
#pragma unroll
    for (int j = 0; j < C::BJ; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, DFH_LPTR(lb + (j * C::RPR + dma_wave * C::ROWS_PER_DMA) * BK),
                                               16, vo, koff, 0, 0);
      vo += b_round;
      asm volatile("" : "+v"(vo));
    }
  };

  const int fa_row = wm * C::WTM + l32;
  const int fb_row = wn * C::WTN + l32;
  typename Op::acc_t acc[C::RN][C::RM];
  // Fragments are double-buffered across the 16-deep k slices: the reads of
  // slice kk+1 are issued before the MFMAs of slice kk, so a wave running alone
  // on its SIMD has its next operands in flight while its MFMAs execute.
  auto compute = [&](auto stc) {
    const uint16_t* la = stA(stc);
    const uint16_t* lb = stB(stc);
    bf16x8 fa[2][C::RM], fb[2][C::RN];
    auto read = [&](int kk, bf16x8 (&ra)[C::RM], bf16x8 (&rb)[C::RN]) {
      const int ch = 2 * kk + hi;
#pragma unroll
      for (int i = 0; i < C::RM; ++i)
        ra[i] = *reinterpret_cast<const bf16x8*>(la + lds_off<CH>(fa_row + i * 32, ch));
#pragma unroll
      for (int i = 0; i < C::RN; ++i)
        rb[i] = *reinterpret_cast<const bf16x8*>(lb + lds_off<CH>(fb_row + i * 32, ch));
    };
    read(0, fa[0], fb[0]);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      // the fences keep the compiler from sinking the reads back to their uses
      __builtin_amdgcn_sched_barrier(0);
      if (kk + 1 < BK / 16) read(kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < C::RN; ++i)
#pragma unroll
        for (int k = 0; k < C::RM; ++k)
          acc[i][k] = Op::mma(fb[kk & 1][i], fa[kk & 1][k], acc[i][k]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  const int KT = K / BK;
  int kb = 0, KTi = KT;  // K steps [kb, kb + KTi) of the current work item
  // Vector-memory ops decrement vmcnt in issue order. The epilogue issues
  // exactly kEpiStores stores after the next tile's prologue DMA, so that
  // tile's first step waits for vmcnt <= kEpiStores (+ the later prologue
  // stages) and leaves the stores in flight. The QKV epilogue (data-dependent
  // store count) waits for zero.
  constexpr int kEpiStoresRaw = (base_epi(EPI) == EPI_QKV) ? -1 : Staged<C, EPI>::value ? Staged<C, EPI>::kVmAfter
                                                                             : C::RN * C::RM * 4;
  constexpr int kWaitBase = ST >= 2 ? (ST - 2) * C::LPS : 0;
  // vmcnt holds at most 63: larger counts fall back to a full wait
  constexpr int kEpiStores = kWaitBase + kEpiStoresRaw < 64 ? kEpiStoresRaw : -1;
  constexpr int kStartWait = kWaitBase + (kEpiStores > 0 ? kEpiStores : 0);
  // bf16 QKV on the single-issue schedules: qkv_epilogue_fixed, counted stores
  constexpr bool kQkvFixed = base_epi(EPI) == EPI_QKV && !is_dq(EPI) && C::SCHED != 2 && C::RN % 2 == 0;
  int qkv_kind = 2;  // the last QKV epilogue's stores: 0 q|k, 1 V (fixed counts), 2 unknown
  static_assert(kStartWait < 64, "vmcnt range");
  // one pipelined K step: k = step index, stage s = k % ST (compile-time)
  // one pipelined K step: k = step index within the item, stage s = k % ST (compile-time)
  auto step = [&](auto stc, int k) {
    constexpr int s = decltype(stc)::value;
    if (k >= KTi) return;  // uniform
    if (k == 0) {
      if constexpr (kQkvFixed) {
        // the QKV epilogue's fixed store counts; every older op (the prologue
        // DMA of stage 0 first) is done once at most this many remain
        constexpr int kQK = kWaitBase + C::RM * C::RN * 4, kV = kWaitBase + C::RM * C::RN * 16;
        if (qkv_kind == 2 || (ST > 2 && KTi < ST - 1)) wait_vm_lgkm0<0>();
        else if (qkv_kind == 0) wait_vm_lgkm0<(kQK < 63 ? kQK : 63)>();
        else wait_vm_lgkm0<(kV < 63 ? kV : 63)>();
      } else if constexpr (kEpiStores >= 0 && ST == 2) {
        wait_vm_lgkm0<kStartWait>();
      } else if constexpr (kEpiStores >= 0) {
        if (KTi >= ST - 1) wait_vm_lgkm0<(kEpiStores >= 0 ? kStartWait : 0)>();
        else wait_vm_lgkm0<0>();
      } else {
        wait_vm_lgkm0<0>();
      }
    } else if (k + ST - 2 >= KTi) {
      wait_vm_lgkm0<0>();   // pipeline drain: exact
    } else {
      wait_vm_lgkm0<(ST >= 2 ? (ST - 2) * C::LPS : 0)>();
    }
    __builtin_amdgcn_s_barrier();
    if (k + ST - 1 < KTi) dma(std::integral_constant<int, (s + ST - 1) % ST>{}, kb + k + ST - 1);
    compute(stc);
  };
  auto kloop = [&]() __attribute__((always_inline)) {
    for (int k0 = 0; k0 < KTi; k0 += ST) {
      step(std::integral_constant<int, 0>{}, k0);
      if constexpr (ST > 1) step(std::integral_constant<int, 1 % ST>{}, k0 + 1);
      if constexpr (ST > 2) step(std::integral_constant<int, 2 % ST>{}, k0 + 2);
      if constexpr (ST > 3) step(std::integral_constant<int, 3 % ST>{}, k0 + 3);
    }
  };
  auto prologue = [&]() __attribute__((always_inline)) {
    dma(std::integral_constant<int, 0>{}, kb);
    if constexpr (ST > 2) { if (1 < KTi) dma(std::integral_constant<int, 1 % ST>{}, kb + 1); }
    if constexpr (ST > 3) { if (2 < KTi) dma(std::integral_constant<int, 2 % ST>{}, kb + 2); }
  };
  // ---- SCHED 2: one wave per SIMD, DMA spread over the MFMAs ----
  // DMA(j) = the A rows of K step j (4 instructions per wave, issued in slice 1
  // of step j - D2) and its B rows (4, in slice 0 of step j - D2 + 1): ST - 1
  // steps ahead, into stage j % ST.
  constexpr int D2 = C::SCHED == 2 ? ST - 1 : 3;  // (other schedules never run this code)
  // vector-memory ops a staged epilogue issues after the next tile's prologue
  // (stores, residual / gate loads) plus the row -> request loads of the next
  // tile's start; -1: unknown or too many to count (then those waits drain fully)
  constexpr int kVm2Raw = (base_epi(EPI) == EPI_QKV || !Staged<C, EPI>::value)
                              ? -1
                              : Staged<C, EPI>::kVmAfter + (Staged<C, EPI>::kRes ? C::RM * Staged<C, EPI>::JB : 0);
  constexpr int kVm2 = kVm2Raw > 63 ? 63 : kVm2Raw;
  constexpr auto epi_n = [](int base) constexpr { return kVm2 < 0 ? 0 : (base + kVm2 > 63 ? 63 : base + kVm2); };
  constexpr int kSteady2 = 8 * (D2 - 2);   // mid-step: DMA(k+2 .. k+D2-1) issued after DMA(k+1)
  constexpr int kStart2 = kSteady2 + 4;    // tile start: DMA(1 .. D2-2) and the A rows of DMA(D2-1)
  bf16x8 g_a[2][C::RM], g_b[2][C::RN];  // fragments of the two 16-deep slices of a step
  // DMA instruction d (0..3) of half h (0: A rows, 1: B rows) of K step ks into stage stc
  auto dma1 = [&](auto stc, int ks, int h, int d) __attribute__((always_inline)) {
    const int koff = ks * BK * 2;
    if (h == 0) {
      uint32_t vo = va + (uint32_t)d * a_round;
      asm volatile("" : "+v"(vo));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, DFH_LPTR(stA(stc) + (d * C::RPR + dma_wave * C::ROWS_PER_DMA) * BK), 16, vo, koff, 0, 0);
    } else {
      uint32_t vo = vb + (uint32_t)d * b_round;
      asm volatile("" : "+v"(vo));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, DFH_LPTR(stB(stc) + (d * C::RPR + dma_wave * C::ROWS_PER_DMA) * BK), 16, vo, koff, 0, 0);
    }
  };
  // fragment read r (0..7) of slice `half` of the step in stage stc, in the order
  // the slice's MFMAs first use them: b0, a0, a1, a2, a3, b1, b2, b3
  auto frag1 = [&](auto stc, int half, int r, bf16x8 (&fa)[C::RM], bf16x8 (&fb)[C::RN])
      __attribute__((always_inline)) {
    const int ch = 2 * half + hi;
    if (r == 0) {
      fb[0] = *reinterpret_cast<const bf16x8*>(stB(stc) + lds_off<CH>(fb_row, ch));
    } else if (r <= C::RM) {
      fa[r - 1] = *reinterpret_cast<const bf16x8*>(stA(stc) + lds_off<CH>(fa_row + (r - 1) * 32, ch));
    } else {
      fb[r - C::RM] = *reinterpret_cast<const bf16x8*>(stB(stc) + lds_off<CH>(fb_row + (r - C::RM) * 32, ch));
    }
  };
  // one 16-deep slice: MFMA t on (fb[t / RM], fa[t % RM]); after MFMA 2j+1 the
  // next slice's fragment read j, after MFMA 4j+2 the DMA instruction j.
  // Z: the tile's first slice, accumulating onto zero.
  auto slice2 = [&](auto zc, bf16x8 (&fa)[C::RM], bf16x8 (&fb)[C::RN], auto&& rd, auto&& dm)
      __attribute__((always_inline)) {
    constexpr bool Z = decltype(zc)::value;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      auto& c = acc[t / C::RM][t % C::RM];
      if constexpr (Z) c = Op::mma(fb[t / C::RM], fa[t % C::RM], typename Op::acc_t{});
      else c = Op::mma(fb[t / C::RM], fa[t % C::RM], c);
      __builtin_amdgcn_sched_barrier(0);
      if (t & 1) {
        rd(t >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if ((t & 3) == 2) {
        dm(t >> 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // mid-step wait of a guarded step: nb = DMA steps issued after DMA(k+1) (0 .. D2-2);
  // epi: the epilogue's memory ops were also issued after it
  auto mid_wait = [&](int nb, bool epi) __attribute__((always_inline)) {
    if (nb >= 2) { if (epi) wait_vm<epi_n(16)>(); else wait_vm<16>(); }
    else if (nb == 1) { if (epi) wait_vm<epi_n(8)>(); else wait_vm<8>(); }
    else { if (epi) wait_vm<epi_n(0)>(); else wait_vm<0>(); }
  };
  // K step k in stage s (= k % ST). Slice 0: MFMAs on g[0], reads of this
  // step's slice 1 into g[1], the B rows of DMA(k+D2-1). Mid-step: this wave's
  // DMA(k+1) has landed (vmcnt), then the barrier makes every wave's visible.
  // Slice 1: MFMAs on g[1], reads of step k+1's slice 0 into g[0], the A rows of
  // DMA(k+D2). Stage (k+D2-1) % ST last held step k-2 and stage (k+D2) % ST step
  // k-1: every wave finished reading them before the barrier of step k-1, resp. k.
  // G: guard the reads / DMA past the last step; epi: see mid_wait; Z: first step.
  auto step2 = [&](auto stc, auto gc, auto zc, int k, bool epi) __attribute__((always_inline)) {
    constexpr int s = decltype(stc)::value;
    constexpr bool G = decltype(gc)::value;
    using Sn = std::integral_constant<int, (s + 1) % ST>;
    using Sa = std::integral_constant<int, (s + D2 - 1) % ST>;
    using Sb = std::integral_constant<int, (s + D2) % ST>;
    if (G && k >= KTi) return;  // uniform
    const bool db = !G || k + D2 - 1 < KTi, rn = !G || k + 1 < KTi, da = !G || k + D2 < KTi;
    slice2(zc, g_a[0], g_b[0], [&](int r) { frag1(stc, 1, r, g_a[1], g_b[1]); },
           [&](int d) { if (db) dma1(Sa{}, kb + k + D2 - 1, 1, d); });
    if constexpr (G) {
      const int nb = KTi - k - 2;
      mid_wait(nb < 0 ? 0 : (nb > D2 - 2 ? D2 - 2 : nb), epi);
    } else {
      wait_vm<kSteady2>();
    }
    __builtin_amdgcn_s_barrier();
    slice2(std::false_type{}, g_a[1], g_b[1], [&](int r) { if (rn) frag1(Sn{}, 0, r, g_a[0], g_b[0]); },
           [&](int d) { if (da) dma1(Sb{}, kb + k + D2, 0, d); });
  };
  // DMA(0 .. D2-2) and the A rows of DMA(D2-1)
  auto prologue2 = [&]() __attribute__((always_inline)) {
    static_for<D2 - 1>([&](auto j) {
      constexpr int J = decltype(j)::value;
      if (J < KTi) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int d = 0; d < 4; ++d) dma1(j, kb + J, h, d);
      }
    });
    if (D2 - 1 < KTi) {
#pragma unroll
      for (int d = 0; d < 4; ++d) dma1(std::integral_constant<int, D2 - 1>{}, kb + D2 - 1, 0, d);
    }
  };
  // the K loop of one item; after_epi: a staged epilogue's memory ops were issued
  // after this item's prologue. Steps 0 .. D2-3 wait for those too; they and the
  // last steps run guarded, the rest in unrolled groups of ST steps.
  auto kloop2 = [&](bool after_epi) __attribute__((always_inline)) {
    using T = std::true_type;
    using F = std::false_type;
    constexpr int P = D2 - 2 > 1 ? D2 - 2 : 1;  // peeled steps
    if (KTi < D2) wait_vm<0>();
    else if (after_epi) wait_vm<epi_n(kStart2)>();
    else wait_vm<kStart2>();
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int r = 0; r < 8; ++r) frag1(std::integral_constant<int, 0>{}, 0, r, g_a[0], g_b[0]);
    step2(std::integral_constant<int, 0>{}, T{}, T{}, 0, after_epi);
    static_for<P - 1>([&](auto j) {
      constexpr int J = decltype(j)::value + 1;
      step2(std::integral_constant<int, J % ST>{}, T{}, F{}, J, after_epi && J <= D2 - 3);
    });
    int k = P;
    for (; k + ST - 1 + D2 < KTi; k += ST)
      static_for<ST>([&](auto j) {
        constexpr int J = decltype(j)::value;
        step2(std::integral_constant<int, (P + J) % ST>{}, F{}, F{}, k + J, false);
      });
    for (; k < KTi; k += ST)
      static_for<ST>([&](auto j) {
        constexpr int J = decltype(j)::value;
        step2(std::integral_constant<int, (P + J) % ST>{}, T{}, F{}, k + J, false);
      });
  };
  // the K piece of a leftover tile this workgroup runs last (piece < 0: none)
  const int tail_tiles = chunk_x - full_x;
  const int piece = (split > 1 && slot < tail_tiles * split) ? slot : -1;
  auto set_item = [&](int jt_or_piece, bool is_piece) -> int {  // returns the tile, sets kb / KTi
    if (!is_piece) { kb = 0; KTi = KT; return xcd * chunk + jt_or_piece; }
    const int kc = jt_or_piece % split;
    kb = kc * KT / split;
    KTi = (kc + 1) * KT / split - kb;
    return xcd * chunk + full_x + jt_or_piece / split;
  };

  int jt = slot;
  int tile = tile_at(jt);
  if (tile >= 0) {
    set_offsets(tile);
    if constexpr (C::SCHED == 2) {
      prologue2();
    } else {
      prologue();
      wait_vm_lgkm0<0>();  // the first tile has no epilogue stores in flight
    }
  }
  bool after_epi = false;
  while (tile >= 0) {
    int m0, n0;
    tile_mn(tile, m0, n0);
#pragma unroll
    for (int i = 0; i < C::RN; ++i)
#pragma unroll
      for (int k = 0; k < C::RM; ++k)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[i][k][t] = 0;
    ResRows<C, EPI> rrows;
    res_rows_load<C, EPI>(a, rrows, m0, M, wm, lane);  // lands during the K loop
    if constexpr (C::SCHED == 2) kloop2(after_epi);
    else kloop();
    // every wave is done with every stage before it is refilled
    wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    StagedOperands<C, EPI> sop;
    if constexpr (Staged<C, EPI>::value) staged_preload<C, EPI>(a, sop, rrows, m0, n0, M, wm, wn, lane, l32, hi);
    // start the next tile's first K steps under this tile's epilogue
    jt += per_xcd;
    const int next = tile_at(jt);
    if (next >= 0) {
      set_offsets(next);
      if constexpr (C::SCHED == 2) prologue2();
      else prologue();
    }
    if constexpr (Staged<C, EPI>::value) {
      // the stage the prologue does not fill (ST - 1); waves split over its A and B buffers
      constexpr int fs = ST - 1;
      uint16_t* region = (wave < C::NW / 2 ? stA(std::integral_constant<int, fs>{})
                                           : stB(std::integral_constant<int, fs>{})) +
                         (wave % (C::NW / 2)) * 32 * C::WTN;
      staged_epilogue<C, EPI>(a, acc, sop, rrows, m0, n0, M, wm, wn, lane, l32, hi, region);
    } else if constexpr (kQkvFixed) {
      qkv_kind = qkv_epilogue_fixed<C>(a, acc, m0, n0, M, wm, wn, l32, hi);
    } else {
      run_epilogue<C, EPI>(a, acc, m0, n0, M, wm, wn, l32, hi);
    }
    after_epi = true;
    tile = next;
  }
  if (piece < 0) return;
  // One K piece of a leftover tile. Its partial sums go to the workspace in MFMA
  // lane layout (one 16-B store per (wave, i, k, quarter, lane)); the workgroup
  // whose piece completes the tile adds all pieces in piece order and runs the
  // tile's epilogue. All pieces of a tile run on one XCD, whose L2 they share:
  // each workgroup waits for its stores to be acknowledged by L2 before it counts
  // itself in with one atomic, and nobody waits for anybody.
  const int tt = piece / split;  // leftover tile within the XCD
  const int tile_p = set_item(piece, true);
  set_offsets(tile_p);
  if constexpr (C::SCHED == 2) {
    prologue2();
  } else {
    prologue();
    wait_vm_lgkm0<0>();
  }
#pragma unroll
  for (int i = 0; i < C::RN; ++i)
#pragma unroll
    for (int k = 0; k < C::RM; ++k)
#pragma unroll
      for (int t = 0; t < 16; ++t) acc[i][k][t] = 0;
  if constexpr (C::SCHED == 2) kloop2(false);
  else kloop();
  using E = typename Op::elem_t;
  auto part_off = [&](int i, int k, int q) {
    return (((((long)wave * C::RN + i) * C::RM + k) * 4 + q) * 64 + lane) * 4;
  };
  // a lane's accumulators belong to one output row; rows at or past M are
  // neither stored nor summed (the epilogue drops them)
  int pm0, pn0;
  tile_mn(tile_p, pm0, pn0);
  auto row_ok = [&](int k) { return pm0 + wm * C::WTM + k * 32 + l32 < M; };
  {
    float* wp = a.ws + kSplitCounters + (long)(xcd * per_xcd + piece) * (BM * BN);
#pragma unroll
    for (int i = 0; i < C::RN; ++i)
#pragma unroll
      for (int k = 0; k < C::RM; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // copy the elements out first: a bit_cast of a vector-element expression reads element 0
          const E e0 = acc[i][k][4 * q], e1 = acc[i][k][4 * q + 1], e2 = acc[i][k][4 * q + 2],
                  e3 = acc[i][k][4 * q + 3];
          if (row_ok(k))
            *reinterpret_cast<float4*>(wp + part_off(i, k, q)) =
              make_float4(__builtin_bit_cast(float, e0), __builtin_bit_cast(float, e1),
                          __builtin_bit_cast(float, e2), __builtin_bit_cast(float, e3));
        }
  }
  // The pieces of a tile are dealt to workgroups xcd, xcd + 8, ...: with the
  // round-robin dispatch of the 8-XCD partition mode they share one L2, where a
  // piece's stores (acknowledged before it counts itself in) are visible to the
  // last arriver's loads. A piece that finds itself on another XCD (hardware
  // register XCC_ID) writes its partial sums back with an agent-scope release
  // fence and marks the tile (counter bits 16..31); the last arriver of a marked
  // tile takes an agent-scope acquire fence before reading the pieces.
  const bool on_xcd = __builtin_amdgcn_s_getreg((3 << 11) | 20) == xcd;  // hwreg(XCC_ID, 0, 4); uniform
  if (!on_xcd) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial sums are in L2
  __syncthreads();                                   // ... and every wave's; LDS reads done too
  unsigned* cnt = reinterpret_cast<unsigned*>(a.ws) + xcd * per_xcd + tt;
  if (tid == 0) {
    const unsigned add = on_xcd ? 1u : 0x10001u;
    const unsigned now = __hip_atomic_fetch_add(cnt, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
    s_flag = (now & 0xffffu) != (unsigned)split ? 0 : (now >> 16) ? 2 : 1;
  }
  __syncthreads();
  if (!s_flag) return;  // uniform
  if (s_flag == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  asm volatile("" ::: "memory");
  if (tid == 0) *cnt = 0u;  // ready for the next launch
  // Last piece in: sum the pieces in piece order, ((p0 + p1) + p2) + ..., the
  // same sum whichever piece arrives last. This workgroup's own piece stays in
  // registers; per 16-value block the pieces before it are added first, then it,
  // then the pieces after it.
  const int own = piece % split;
  const float* wbase = a.ws + kSplitCounters + (long)(xcd * per_xcd + tt * split) * (BM * BN);
  auto load_block = [&](int kc, int i, int k, E (&x)[16]) {
    const float* wp = wbase + (long)kc * (BM * BN);
    const bool ok = row_ok(k);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = ok ? *reinterpret_cast<const float4*>(wp + part_off(i, k, q)) : make_float4(0.f, 0.f, 0.f, 0.f);
      x[4 * q] = __builtin_bit_cast(E, v.x);
      x[4 * q + 1] = __builtin_bit_cast(E, v.y);
      x[4 * q + 2] = __builtin_bit_cast(E, v.z);
      x[4 * q + 3] = __builtin_bit_cast(E, v.w);
    }
  };
#pragma unroll
  for (int i = 0; i < C::RN; ++i)
#pragma unroll
    for (int k = 0; k < C::RM; ++k) {
      if (own > 0) {
        E t[16], x[16];
        load_block(0, i, k, t);
        for (int kc = 1; kc < own; ++kc) {
          load_block(kc, i, k, x);
#pragma unroll
          for (int v = 0; v < 16; ++v) t[v] = t[v] + x[v];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][k][v] = t[v] + acc[i][k][v];
      }
      for (int kc = own + 1; kc < split; ++kc) {
        E x[16];
        load_block(kc, i, k, x);
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][k][v] = acc[i][k][v] + x[v];
      }
    }
  {
    int m0, n0;
    tile_mn(tile_p, m0, n0);
    if constexpr (Staged<C, EPI>::value) {
      StagedOperands<C, EPI> sop;
      ResRows<C, EPI> rrows;
      res_rows_load<C, EPI>(a, rrows, m0, M, wm, lane);
      staged_preload<C, EPI>(a, sop, rrows, m0, n0, M, wm, wn, lane, l32, hi);
      constexpr int fs = ST - 1;
      uint16_t* region = (wave < C::NW / 2 ? stA(std::integral_constant<int, fs>{})
                                           : stB(std::integral_constant<int, fs>{})) +
                         (wave % (C::NW / 2)) * 32 * C::WTN;
      staged_epilogue<C, EPI>(a, acc, sop, rrows, m0, n0, M, wm, wn, lane, l32, hi, region);
    } else {
      run_epilogue<C, EPI>(a, acc, m0, n0, M, wm, wn, l32, hi);
    }
  }
}

int g_num_cus = 0;

int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) == hipSuccess) g_num_cus = p.multiProcessorCount;
    if (g_num_cus <= 0) g_num_cus = 256;
  }
  return g_num_cus;
}

template <class C, class Op, int EPI>
hipError_t launch(const GemmArgs& a_in, hipStream_t s) {
  auto kern = gemm_mfma_kernel<C, Op, EPI>;
  const long tiles_upper = (long)((a_in.M + C::BM - 1) / C::BM) * (a_in.N / C::BN);
  const long full = (long)num_cus() * C::WG_PER_CU;
  GemmArgs a = a_in;
  // the K-split needs the counters and a partial-sum tile per workgroup
  if (a.ws && (full > kSplitCounters || a.ws_elems < kSplitCounters + full * C::BM * C::BN))
    a.ws = nullptr;
  // Fewer tiles than resident workgroups: with a workspace the whole grid runs
  // and the idle workgroups take K pieces of the tiles (the split of a partial
  // last round, here the only round); without one the grid shrinks to the tiles.
  long grid = full;
  if (tiles_upper < grid && !a.ws) grid = ((tiles_upper + 7) / 8) * 8;
  if (grid < 8) grid = 8;
  dfh_launch(kern, dim3((unsigned)grid), dim3(C::THREADS), 0, s, a);
  return hipGetLastError();
}

// tile configurations: (BM, BN, BK, stages, wave grid)
using T0 = Cfg<256, 256, 64, 2, 2, 4>;  // 8 waves, 128x64 per wave, 128 KB LDS
using T1 = Cfg<256, 256, 32, 4, 2, 4>;  // 8 waves, 4 stages of BK 32, 128 KB
using T2 = Cfg<128, 128, 64, 2, 2, 2>;  // 4 waves, 64 KB: two workgroups per CU
using T3 = Cfg<64, 64, 64, 2, 2, 2>;    // small problems
using T4 = Cfg<256, 128, 64, 2, 2, 2>;  // 4 waves, 128x64 per wave, 96 KB
using T5 = Cfg<128, 256, 32, 3, 2, 2>;  // 4 waves, 64x128 per wave, 72 KB: two per CU
using T6 = Cfg<256, 128, 64, 3, 2, 2>;  // 4 waves, 3 stages, 144 KB
using T7 = Cfg<128, 128, 32, 4, 2, 2>;  // 4 waves, 4 stages of BK 32, 64 KB: two per CU
using T8 = Cfg<256, 256, 64, 2, 2, 4, 1>;  // T0 with the DMA of a step issued by one half
using T9 = Cfg<256, 256, 32, 5, 2, 2, 2>;  // 4 waves, 128x128 per wave (AGPRs), DMA spread over the MFMAs, 160 KB
// at most 128 rows (a decode-sized batch): one row block, narrow column blocks
// and K pieces spread the weights over the whole chip; two workgroups per CU.
// At most 8 pieces of at least 4 K steps per tile: at 68 rows, K = 4096 runs
// faster as 8 pieces of 8 K steps than as 16 of 4 (the last piece's sum and
// epilogue cost per piece), while K = 1024 is fastest as 4 pieces of 4.
using T10 = Cfg<128, 32, 64, 4, 4, 1, 0, 8, 4>;  // 4 waves, 32x32 per wave, 80 KB
using T11 = Cfg<128, 64, 64, 3, 4, 1, 0, 8, 4>;  // 4 waves, 32x64 per wave (RoPE pairs of the QKV epilogue), 72 KB
constexpr int kNumTiles = 12;
const int kTileBM[kNumTiles] = {T0::BM, T1::BM, T2::BM, T3::BM, T4::BM,  T5::BM,
                                T6::BM, T7::BM, T8::BM, T9::BM, T10::BM, T11::BM};
const int kTileBN[kNumTiles] = {T0::BN, T1::BN, T2::BN, T3::BN, T4::BN,  T5::BN,
                                T6::BN, T7::BN, T8::BN, T9::BN, T10::BN, T11::BN};
const int kTileBK[kNumTiles] = {T0::BK, T1::BK, T2::BK, T3::BK, T4::BK,  T5::BK,
                                T6::BK, T7::BK, T8::BK, T9::BK, T10::BK, T11::BK};
const int kTileWTN[kNumTiles] = {T0::WTN, T1::WTN, T2::WTN, T3::WTN, T4::WTN,  T5::WTN,
                                 T6::WTN, T7::WTN, T8::WTN, T9::WTN, T10::WTN, T11::WTN};

template <class Op, int EPI>
hipError_t dispatch_tiles(const GemmArgs& a, hipStream_t s, int tile) {
  switch (tile) {
    case 0: return launch<T0, Op, EPI>(a, s);
    case 1: return launch<T1, Op, EPI>(a, s);
    case 2: return launch<T2, Op, EPI>(a, s);
    case 3: return launch<T3, Op, EPI>(a, s);
    case 4: return launch<T4, Op, EPI>(a, s);
    case 5: return launch<T5, Op, EPI>(a, s);
    case 6: return launch<T6, Op, EPI>(a, s);
    case 7: return launch<T7, Op, EPI>(a, s);
    case 8: return launch<T8, Op, EPI>(a, s);
    case 9: return launch<T9, Op, EPI>(a, s);
    case 10: return launch<T10, Op, EPI>(a, s);
    case 11: return launch<T11, Op, EPI>(a, s);
    default: return hipErrorInvalidValue;
  }
}

int pick_tile(const GemmArgs& a) {
  const long cus = num_cus();
  if (a.M <= 128 && a.N % 32 == 0 && a.K % 64 == 0) return 10;
  // up to 2048 rows and 2048..8192 columns (the latent tail's fc1 and q at 1024
  // rows): 128x64 tiles and their K pieces fill the chip; at 1024 x 4096 x 1024
  // 13.8 us against 20.5 on 128x128 tiles
  if (a.M <= 2048 && a.N >= 2048 && a.N <= 8192 && a.N % 64 == 0 && a.K % 64 == 0) return 11;
  const long t0 = (long)((a.M + 255) / 256) * (a.N / 256);
  if (a.N % 256 == 0 && a.K % 64 == 0 && t0 >= 2 * cus) return 8;
  if (a.N % 128 == 0 && a.K % 64 == 0 && (long)((a.M + 127) / 128) * (a.N / 128) >= cus) return 2;
  return 3;
}

}  // namespace

int cu_count() { return num_cus(); }

hipError_t gemm_bf16(const GemmArgs& a, int epi, hipStream_t s, int tile) {
  if (a.K <= 0 || a.N <= 0 || a.M < 0 || a.K % 32 != 0) return hipErrorInvalidValue;
  if (a.M == 0) return hipSuccess;  // a.M is the host upper bound of rows
  if (tile < 0) tile = pick_tile(a);
  if (tile < 0 || tile >= kNumTiles) return hipErrorInvalidValue;
  if (epi == EPI_QKV && kTileWTN[tile] < 64) tile = a.M <= 2048 ? 11 : 2;  // RoPE pairs need a 64-column wave tile
  if (a.N % kTileBN[tile] != 0 || a.K % kTileBK[tile] != 0) return hipErrorInvalidValue;
  if (epi == EPI_QKV && (a.hidden % kTileBN[tile] != 0 || a.head_dim != 64)) return hipErrorInvalidValue;
  // element offsets are 32-bit
  if ((long)a.M * a.lda >= (1L << 31) || (long)a.N * a.ldb >= (1L << 31)) return hipErrorInvalidValue;
  (void)kTileBM;
  switch (epi) {
    case EPI_BIAS: return dispatch_tiles<OpBf16, EPI_BIAS>(a, s, tile);
    case EPI_GELU: return dispatch_tiles<OpBf16, EPI_GELU>(a, s, tile);
    case EPI_SILU: return dispatch_tiles<OpBf16, EPI_SILU>(a, s, tile);
    case EPI_GATE_RES: return dispatch_tiles<OpBf16, EPI_GATE_RES>(a, s, tile);
    case EPI_QKV: return dispatch_tiles<OpBf16, EPI_QKV>(a, s, tile);
    case EPI_F32: return dispatch_tiles<OpBf16, EPI_F32>(a, s, tile);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemm_i8(const GemmArgs& a_bytes, int epi, hipStream_t s, int tile) {
  // byte-sized K and leading dimensions -> 16-bit units of the shared tile machinery
  if (a_bytes.K <= 0 || a_bytes.K % 64 != 0 || a_bytes.lda % 16 != 0 || a_bytes.ldb % 16 != 0)
    return hipErrorInvalidValue;
  if (a_bytes.N <= 0 || a_bytes.M < 0) return hipErrorInvalidValue;
  if (a_bytes.M == 0) return hipSuccess;
  GemmArgs a = a_bytes;
  a.K = a_bytes.K / 2;
  a.lda = a_bytes.lda / 2;
  a.ldb = a_bytes.ldb / 2;
  if (tile < 0) {
    // int8 takes the 256x256 tile from one full round of its tiles on (the bf16
    // heuristic waits for two): at M = 16384, N = 1024 it runs 9-18 % faster
    // than two 128x128 workgroups per CU
    const long t0 = (long)((a.M + 255) / 256) * (a.N / 256);
    tile = (a.N % 256 == 0 && a.K % 64 == 0 && t0 >= num_cus()) ? 8 : pick_tile(a);
  }
  if (tile < 0 || tile >= kNumTiles) return hipErrorInvalidValue;
  if (epi == EPI_DQ_QKV && kTileWTN[tile] < 64) tile = a.M <= 2048 ? 11 : 2;  // RoPE pairs need a 64-column wave tile
  if (a.N % kTileBN[tile] != 0 || a.K % kTileBK[tile] != 0) return hipErrorInvalidValue;
  if (epi == EPI_DQ_QKV && (a.hidden % kTileBN[tile] != 0 || a.head_dim != 64)) return hipErrorInvalidValue;
  if (is_dq(epi) && (!a.sx || !a.sw)) return hipErrorInvalidValue;
  if ((long)a.M * a.lda >= (1L << 31) || (long)a.N * a.ldb >= (1L << 31)) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_I32: return dispatch_tiles<OpI8, EPI_I32>(a, s, tile);
    case EPI_DQ: return dispatch_tiles<OpI8, EPI_DQ>(a, s, tile);
    case EPI_DQ_GELU: return dispatch_tiles<OpI8, EPI_DQ_GELU>(a, s, tile);
    case EPI_DQ_GATE_RES: return dispatch_tiles<OpI8, EPI_DQ_GATE_RES>(a, s, tile);
    case EPI_DQ_QKV: return dispatch_tiles<OpI8, EPI_DQ_QKV>(a, s, tile);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dfh
