// Varlen attention with the implicit FM mask, head_dim 64, bf16 MFMA.
//
// Request i occupies packed rows [cu_rows[i], cu_rows[i] + c_i + P): c_i history
// rows then P latent rows. The mask of DotsModel._build_fm_attn_mask
// (nanovllm_dots/models/dots/native/model.py:57-75) without its padding gap is a
// key prefix per query row r:
//     visible keys = [0, r+1)        for r <  c_i - 1   (causal history)
//                  = [0, c_i + P)    for r >= c_i - 1   (last hidden row + latents)
// so no mask tensor is read. softmax(q k^T / 8) v with an online (flash) softmax.
//
// Work split: one workgroup = 128 query rows of one (request, head); wave w owns
// 32 rows. Per 64-key tile the wave computes S^T = K Q^T (32 keys x 32 queries
// per MFMA block): a lane then holds 32 key scores of ONE query, so the row
// max/sum need a single cross-lane exchange (lane ^ 32), and the probabilities
// are already in the B-operand layout of O^T += V^T P^T. V arrives transposed
// (V^T [H, tokens], written by the QKV GEMM epilogue) so its A-operand
// fragments are contiguous LDS reads.
#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

constexpr int BQ = 128;    // query rows per workgroup
constexpr int BKV = 64;    // keys per tile
constexpr int HD = 64;     // head dim
constexpr int LDS_K = HD + 8;    // K tile row: 64 d + pad
constexpr int LDS_V = BKV + 8;   // V^T tile row: 64 keys + pad

__global__ void __launch_bounds__(256, 2)
fm_attention_kernel(const uint16_t* __restrict__ qk, long ldqk, const uint16_t* __restrict__ vt,
                    long ld_vt, uint16_t* __restrict__ out, long ldo, const int* __restrict__ cu_rows,
                    const int* __restrict__ cu_vt, const int* __restrict__ hist_len, int patch,
                    int heads, float scale_log2) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * LDS_K];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][HD * LDS_V];

  const int req = blockIdx.z, h = blockIdx.y;
  const int nq = gridDim.x;
  const int qt = nq - 1 - (int)blockIdx.x;  // longest (last) query tiles first
  const int c = hist_len[req];
  const int T = c + patch;
  const int q0 = qt * BQ;
  if (q0 >= T) return;
  const int row0 = cu_rows[req];
  const int vcol0 = cu_vt[req];
  const int H = heads * HD;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;

  const int r_last = min(q0 + BQ - 1, T - 1);
  const int kmax = (r_last >= c - 1) ? T : r_last + 1;  // keys needed by this workgroup
  const int ntiles = (kmax + BKV - 1) / BKV;

  // this lane's query (request-local) and its visible-key limit
  const int q = q0 + wave * 32 + l32;
  const int qc = q < T ? q : T - 1;
  const int lim = (qc < c - 1) ? qc + 1 : T;
  // keys needed by this wave
  const int wq_last = min(q0 + wave * 32 + 31, T - 1);
  const int wave_kmax = (q0 + wave * 32 >= T) ? 0 : ((wq_last >= c - 1) ? T : wq_last + 1);

  // Q fragments (B operand): Q[q][16*kk + 8*hi .. +8]
  bf16x8 qf[4];
  {
    const uint16_t* qp = qk + (long)(row0 + qc) * ldqk + h * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qp + 16 * kk);
  }

  // cooperative tile loads: K tile 64 keys x 128 B, V^T tile 64 d x 128 B; 2+2 chunks/thread
  auto load_tile = [&](int t, uint4* rk, uint4* rv) {
    const int k0 = t * BKV;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int idx = tid + cc * 256;
      const int r = idx >> 3, col = (idx & 7) * 8;
      int key = k0 + r;
      key = key < T ? key : T - 1;
      rk[cc] = *reinterpret_cast<const uint4*>(qk + (long)(row0 + key) * ldqk + H + h * HD + col);
      rv[cc] = *reinterpret_cast<const uint4*>(vt + (long)(h * HD + r) * ld_vt + vcol0 + k0 + col);
    }
  };
  auto store_tile = [&](int buf, const uint4* rk, const uint4* rv) {
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int idx = tid + cc * 256;
      const int r = idx >> 3, col = (idx & 7) * 8;
      *reinterpret_cast<uint4*>(&Ks[buf][r * LDS_K + col]) = rk[cc];
      *reinterpret_cast<uint4*>(&Vs[buf][r * LDS_V + col]) = rv[cc];
    }
  };

  floatx16 o[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[b][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  uint4 rk[2], rv[2];
  load_tile(0, rk, rv);
  store_tile(0, rk, rv);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1, rk, rv);
    const int k0 = t * BKV;
    if (k0 < wave_kmax) {
      // S^T blocks: keys k0 + 32*kb + (8*(v/4) + 4*hi + v%4), query = q
      floatx16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
        const uint16_t* kp = &Ks[cur][(kb * 32 + l32) * LDS_K + 8 * hi];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          bf16x8 kf = *reinterpret_cast<const bf16x8*>(kp + 16 * kk);
          s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kb], 0, 0, 0);
        }
      }
      // mask + running max
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + kb * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
          const float sv = key < lim ? s[kb][v] * scale_log2 : -INFINITY;
          s[kb][v] = sv;
          mx = fmaxf(mx, sv);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = exp2f(s[kb][v] - m_new);
          s[kb][v] = p;
          psum += p;
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[b][v] *= alpha;
      // O^T[d][q] += V^T[d][keys] P^T[keys][q]; k-step (kb, half) covers keys
      // kb*32 + 16*half + [0,16): lane holds 8*(v/4) + 4*hi + v%4 for v in [8half, 8half+8)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          bf16x8 pf;
#pragma unroll
          for (int j = 0; j < 8; ++j) pf[j] = (__bf16)s[kb][8 * half + j];
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const uint16_t* vp = &Vs[cur][(db * 32 + l32) * LDS_V + kb * 32 + 16 * half + 4 * hi];
            uint2 lo = *reinterpret_cast<const uint2*>(vp);
            uint2 up = *reinterpret_cast<const uint2*>(vp + 8);
            uint4 u = make_uint4(lo.x, lo.y, up.x, up.y);
            bf16x8 vf = *reinterpret_cast<bf16x8*>(&u);
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
          }
        }
    }
    if (t + 1 < ntiles) store_tile(cur ^ 1, rk, rv);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (q < T) {
    const float inv = 1.0f / l_tot;
    uint16_t* op = out + (long)(row0 + q) * ldo + h * HD;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hi;
        *reinterpret_cast<uint2*>(op + d) =
            pack4(o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                  o[db][4 * g + 3] * inv);
      }
  }
}

}  // namespace

hipError_t fm_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt,
                        uint16_t* out, long ldo, const int* cu_rows, const int* cu_vt,
                        const int* hist_len, int n_req, int patch, int heads, int max_T,
                        hipStream_t s) {
  if (n_req <= 0) return hipSuccess;
  const float scale_log2 = 0.125f * 1.4426950408889634f;  // head_dim^-0.5 * log2(e)
  dim3 grid((max_T + BQ - 1) / BQ, heads, n_req);
  dfh_launch(fm_attention_kernel, grid, dim3(256), 0, s, qk, ldqk, vt, ld_vt, out, ldo,
                     cu_rows, cu_vt, hist_len, patch, heads, scale_log2);
  return hipGetLastError();
}

}  // namespace dfh
