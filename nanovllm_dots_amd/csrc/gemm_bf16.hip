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
// XCD-contiguous chunks so the row tiles that share A live in one XCD's L2,
// LDS double buffering with one barrier per 64-wide K step, global loads for
// step k+1 issued before the MFMAs of step k.
#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded LDS row (elements): 144 B keeps 16-B reads conflict-free

template <int BM, int BN, int WM, int WN>
struct Cfg {
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int WTM = BM / WM;  // wave tile rows (activations)
  static constexpr int WTN = BN / WN;  // wave tile cols (outputs)
  static constexpr int RM = WTM / 32;
  static constexpr int RN = WTN / 32;
  static constexpr int A_CHUNKS = BM * BK / 8 / THREADS;  // 16-B chunks per thread per K step
  static constexpr int B_CHUNKS = BN * BK / 8 / THREADS;
  static constexpr int LDS_BYTES = 2 * (BM + BN) * LDK * 2;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  static_assert((BM * BK / 8) % THREADS == 0 && (BN * BK / 8) % THREADS == 0, "load split");
};

template <int EPI>
__device__ __forceinline__ void epilogue_store4(const GemmArgs& a, int m, int n, const float* v4) {
  // v4: 4 accumulators for columns n..n+3 of row m (m < M checked by caller)
  float y[4];
  if (a.bias) {
    uint2 bb = *reinterpret_cast<const uint2*>(a.bias + n);
    float b[4];
    unpack4(bb, b);
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = v4[t] + b[t];
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = v4[t];
  }
  if constexpr (EPI == EPI_F32) {
    float4 o = make_float4(y[0], y[1], y[2], y[3]);
    *reinterpret_cast<float4*>(a.Cf + (long)m * a.ldc + n) = o;
    return;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = rbf(y[t]);
  if constexpr (EPI == EPI_GELU) {
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = gelu_tanh_f(y[t]);
  }
  if constexpr (EPI == EPI_GATE_RES) {
    const int req = a.row_req[m];
    float g[4], x[4];
    unpack4(*reinterpret_cast<const uint2*>(a.gate + (long)req * a.ld_gate + n), g);
    uint16_t* cp = a.C + (long)m * a.ldc + n;
    unpack4(*reinterpret_cast<const uint2*>(cp), x);
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = x[t] + rbf(g[t] * y[t]);
  }
  *reinterpret_cast<uint2*>(a.C + (long)m * a.ldc + n) = pack4(y[0], y[1], y[2], y[3]);
}

template <int BM, int BN, int WM, int WN, int EPI>
__global__ void __launch_bounds__(64 * WM * WN, 1)
gemm_bf16_kernel(GemmArgs a) {
  using C = Cfg<BM, BN, WM, WN>;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* As = smem;                       // [2][BM][LDK]
  uint16_t* Bs = smem + 2 * BM * LDK;        // [2][BN][LDK]

  const int M = a.M_dev ? *a.M_dev : a.M;
  const int N = a.N, K = a.K;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  if (total == 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, hi = lane >> 5;

  // XCD-contiguous tile walk: workgroups with equal blockIdx.x % 8 share an XCD.
  const int nxcd = 8;
  const int xcd = blockIdx.x % nxcd;
  const int slot = blockIdx.x / nxcd;
  const int per_xcd = gridDim.x / nxcd;
  const int chunk = (total + nxcd - 1) / nxcd;

  for (int j = slot; j < chunk; j += per_xcd) {
    const int tile = xcd * chunk + j;
    if (tile >= total) break;
    const int tm = tile / tiles_n, tn = tile % tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    // per-thread global chunk offsets in elements (fixed over K; rows past M clamp to M-1)
    int a_off[C::A_CHUNKS], a_lds[C::A_CHUNKS];
#pragma unroll
    for (int c = 0; c < C::A_CHUNKS; ++c) {
      int idx = tid + c * C::THREADS;
      int row = idx >> 3, col = (idx & 7) * 8;
      int gm = m0 + row;
      gm = gm < M ? gm : M - 1;
      a_off[c] = gm * (int)a.lda + col;
      a_lds[c] = row * LDK + col;
    }
    int b_off[C::B_CHUNKS], b_lds[C::B_CHUNKS];
#pragma unroll
    for (int c = 0; c < C::B_CHUNKS; ++c) {
      int idx = tid + c * C::THREADS;
      int row = idx >> 3, col = (idx & 7) * 8;
      b_off[c] = (n0 + row) * (int)a.ldb + col;
      b_lds[c] = row * LDK + col;
    }

    floatx16 acc[C::RN][C::RM];
#pragma unroll
    for (int i = 0; i < C::RN; ++i)
#pragma unroll
      for (int k = 0; k < C::RM; ++k)
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[i][k][t] = 0.f;

    uint4 ra[C::A_CHUNKS], rb[C::B_CHUNKS];
#pragma unroll
    for (int c = 0; c < C::A_CHUNKS; ++c) ra[c] = *reinterpret_cast<const uint4*>(a.A + a_off[c]);
#pragma unroll
    for (int c = 0; c < C::B_CHUNKS; ++c) rb[c] = *reinterpret_cast<const uint4*>(a.B + b_off[c]);
    __syncthreads();  // previous tile's LDS readers are done
#pragma unroll
    for (int c = 0; c < C::A_CHUNKS; ++c) *reinterpret_cast<uint4*>(As + a_lds[c]) = ra[c];
#pragma unroll
    for (int c = 0; c < C::B_CHUNKS; ++c) *reinterpret_cast<uint4*>(Bs + b_lds[c]) = rb[c];
    __syncthreads();

    const int KT = K / BK;
    for (int kt = 0; kt < KT; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < KT) {
        const int koff = (kt + 1) * BK;
#pragma unroll
        for (int c = 0; c < C::A_CHUNKS; ++c) ra[c] = *reinterpret_cast<const uint4*>(a.A + a_off[c] + koff);
#pragma unroll
        for (int c = 0; c < C::B_CHUNKS; ++c) rb[c] = *reinterpret_cast<const uint4*>(a.B + b_off[c] + koff);
      }
      const uint16_t* as = As + cur * BM * LDK + (wm * C::WTM + l32) * LDK + hi * 8;
      const uint16_t* bs = Bs + cur * BN * LDK + (wn * C::WTN + l32) * LDK + hi * 8;
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8 fa[C::RM], fb[C::RN];
#pragma unroll
        for (int i = 0; i < C::RM; ++i)
          fa[i] = *reinterpret_cast<const bf16x8*>(as + i * 32 * LDK + kk * 16);
#pragma unroll
        for (int i = 0; i < C::RN; ++i)
          fb[i] = *reinterpret_cast<const bf16x8*>(bs + i * 32 * LDK + kk * 16);
#pragma unroll
        for (int i = 0; i < C::RN; ++i)
#pragma unroll
          for (int k = 0; k < C::RM; ++k)
            acc[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[i], fa[k], acc[i][k], 0, 0, 0);
      }
      if (kt + 1 < KT) {
        const int nxt = cur ^ 1;
#pragma unroll
        for (int c = 0; c < C::A_CHUNKS; ++c)
          *reinterpret_cast<uint4*>(As + nxt * BM * LDK + a_lds[c]) = ra[c];
#pragma unroll
        for (int c = 0; c < C::B_CHUNKS; ++c)
          *reinterpret_cast<uint4*>(Bs + nxt * BN * LDK + b_lds[c]) = rb[c];
      }
      __syncthreads();
    }

    // ---- epilogue: block (i, k) holds D[n][m], lane: m = l32, n = 8*(v/4) + 4*hi + v%4
    if constexpr (EPI == EPI_QKV) {
      const int H = a.hidden;
      const int region = n0 / H;  // 0 q, 1 k, 2 v (BN divides H)
#pragma unroll
      for (int k = 0; k < C::RM; ++k) {
        const int m = m0 + wm * C::WTM + k * 32 + l32;
        const bool valid = m < M;
        const int mm = valid ? m : M - 1;
        if (region == 2) {
          const int col = a.vt_col[mm];
#pragma unroll
          for (int i = 0; i < C::RN; ++i) {
            const int nb = n0 + wn * C::WTN + i * 32 - 2 * H;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int n = nb + 8 * (v >> 2) + 4 * hi + (v & 3);
              float y = acc[i][k][v] + (a.bias ? bf2f(a.bias[n + 2 * H]) : 0.f);
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
            x0[v] = rbf(acc[i][k][v] + b0);
            x1[v] = rbf(acc[i + 1][k][v] + b1);
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
          if (a.rope_cos) {
            const float* cs = a.rope_cos + (long)pos * 32;
            const float* sn = a.rope_sin + (long)pos * 32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int d = 8 * (v >> 2) + 4 * hi + (v & 3);
              const float c = cs[d], s = sn[d];
              const float r0 = __fadd_rn(__fmul_rn(x0[v], c), __fmul_rn(-x1[v], s));
              const float r1 = __fadd_rn(__fmul_rn(x1[v], c), __fmul_rn(x0[v], s));
              x0[v] = r0;
              x1[v] = r1;
            }
          }
          if (valid) {
            uint16_t* cp = a.C + (long)m * a.ldc + nb;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int d = 8 * g + 4 * hi;
              *reinterpret_cast<uint2*>(cp + d) =
                  pack4(x0[4 * g], x0[4 * g + 1], x0[4 * g + 2], x0[4 * g + 3]);
              *reinterpret_cast<uint2*>(cp + 32 + d) =
                  pack4(x1[4 * g], x1[4 * g + 1], x1[4 * g + 2], x1[4 * g + 3]);
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < C::RM; ++k) {
        const int m = m0 + wm * C::WTM + k * 32 + l32;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < C::RN; ++i) {
          const int nb = n0 + wn * C::WTN + i * 32;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float v4[4] = {acc[i][k][4 * g], acc[i][k][4 * g + 1], acc[i][k][4 * g + 2],
                           acc[i][k][4 * g + 3]};
            epilogue_store4<EPI>(a, m, nb + 8 * g + 4 * hi, v4);
          }
        }
      }
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

template <int BM, int BN, int WM, int WN, int EPI>
hipError_t launch(const GemmArgs& a, hipStream_t s) {
  using C = Cfg<BM, BN, WM, WN>;
  auto kern = gemm_bf16_kernel<BM, BN, WM, WN, EPI>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const long tiles_upper = (long)((a.M + BM - 1) / BM) * (a.N / BN);
  const int wg_per_cu = (160 * 1024) / C::LDS_BYTES >= 2 ? 2 : 1;
  long grid = (long)num_cus() * wg_per_cu;
  if (tiles_upper < grid) grid = ((tiles_upper + 7) / 8) * 8;
  if (grid < 8) grid = 8;
  dfh_launch(kern, dim3((unsigned)grid), dim3(C::THREADS), C::LDS_BYTES, s, a);
  return hipGetLastError();
}

template <int EPI>
hipError_t dispatch_tiles(const GemmArgs& a, hipStream_t s, int tile) {
  switch (tile) {
    case 0: return launch<256, 256, 2, 2, EPI>(a, s);
    case 1: return launch<256, 128, 2, 2, EPI>(a, s);
    case 2: return launch<128, 128, 2, 2, EPI>(a, s);
    case 3: return launch<64, 64, 2, 2, EPI>(a, s);
    default: return hipErrorInvalidValue;
  }
}

const int kTileBN[4] = {256, 128, 128, 64};
const int kTileBM[4] = {256, 256, 128, 64};

}  // namespace

hipError_t gemm_bf16(const GemmArgs& a, int epi, hipStream_t s, int tile) {
  if (a.K % BK != 0 || a.K <= 0 || a.N <= 0 || a.M < 0) return hipErrorInvalidValue;
  if (a.M == 0) return hipSuccess;  // a.M is the host upper bound of rows
  if (tile < 0) {
    // heuristic: big tiles for big problems, keep >= ~1 wave of tiles on the chip
    const long t0 = (long)((a.M + 255) / 256) * (a.N / 256);
    if (a.N % 256 == 0 && t0 >= 2L * num_cus()) tile = 0;
    else if (a.N % 128 == 0 && (long)((a.M + 255) / 256) * (a.N / 128) >= num_cus()) tile = 1;
    else if (a.N % 128 == 0 && (long)((a.M + 127) / 128) * (a.N / 128) >= num_cus() / 2) tile = 2;
    else tile = 3;
  }
  if (tile < 0 || tile > 3) return hipErrorInvalidValue;
  if (a.N % kTileBN[tile] != 0) return hipErrorInvalidValue;
  if (epi == EPI_QKV) {
    if (tile == 3) tile = 2;  // RoPE pairs need a 64-column wave tile
    if (a.N % kTileBN[tile] != 0 || a.hidden % kTileBN[tile] != 0 || a.head_dim != 64)
      return hipErrorInvalidValue;
  }
  // element offsets are 32-bit
  if ((long)a.M * a.lda >= (1L << 31) || (long)a.N * a.ldb >= (1L << 31)) return hipErrorInvalidValue;
  (void)kTileBM;
  switch (epi) {
    case EPI_BIAS: return dispatch_tiles<EPI_BIAS>(a, s, tile);
    case EPI_GELU: return dispatch_tiles<EPI_GELU>(a, s, tile);
    case EPI_GATE_RES: return dispatch_tiles<EPI_GATE_RES>(a, s, tile);
    case EPI_QKV: return dispatch_tiles<EPI_QKV>(a, s, tile);
    case EPI_F32: return dispatch_tiles<EPI_F32>(a, s, tile);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dfh
