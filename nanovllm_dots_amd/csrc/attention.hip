// Varlen attention with the implicit FM mask, head_dim 64, bf16 MFMA.
//
// Each sequence is described by an AttnSeq (dfh_kernels.h): its keys are rows
// kv_row0 + [0, kv_len) of the q|k buffer (V^T columns vt_col0 + [0, kv_len)),
// and query q (in [q_begin, q_end)) sees the key prefix
//     [0, q+1)       for q <  causal_end     (causal history)
//     [0, kv_len)    for q >= causal_end     (last hidden row + latent rows)
// For a packed FM request (c history rows then P latent rows, no padding gap)
// this is DotsModel._build_fm_attn_mask (nanovllm_dots/models/dots/native/
// model.py:57-75) with causal_end = c - 1, kv_len = c + P; a cached prefix pass
// is all-causal from a nonzero q_begin. No mask tensor is read.
// softmax(q k^T / 8) v with an online (flash) softmax.
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
seq_attention_kernel(const uint16_t* __restrict__ qk, long ldqk, const uint16_t* __restrict__ vt,
                     long ld_vt, uint16_t* __restrict__ out, long ldo, const AttnSeq* __restrict__ seqs,
                     int heads, float scale_log2) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * LDS_K];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][HD * LDS_V];

  const AttnSeq sq = seqs[blockIdx.z];
  const int h = blockIdx.y;
  const int nq = gridDim.x;
  const int qt = nq - 1 - (int)blockIdx.x;  // longest (last) query tiles first
  const int q0 = sq.q_begin + qt * BQ;
  if (q0 >= sq.q_end) return;
  const int T = sq.kv_len;           // keys of full rows
  const int cend = sq.causal_end;    // queries below this are causal
  const int H = heads * HD;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;

  // visible keys of query q: [0, q+1) below cend, [0, T) from cend on
  auto limit = [&](int q) { return q < cend ? q + 1 : T; };
  const int r_last = min(q0 + BQ, sq.q_end) - 1;
  const int kmax = limit(r_last);  // keys needed by this workgroup (limit is monotone)
  const int ntiles = (kmax + BKV - 1) / BKV;

  // this lane's query and its visible-key limit
  const int q = q0 + wave * 32 + l32;
  const int qc = q < sq.q_end ? q : sq.q_end - 1;
  const int lim = limit(qc);
  // keys needed by this wave
  const int wq_first = q0 + wave * 32;
  const int wave_kmax = wq_first >= sq.q_end ? 0 : limit(min(wq_first + 31, sq.q_end - 1));

  // Q fragments (B operand): Q[q][16*kk + 8*hi .. +8]
  bf16x8 qf[4];
  {
    const uint16_t* qp = qk + (long)(sq.q_row0 + qc) * ldqk + h * HD + 8 * hi;
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
      rk[cc] = *reinterpret_cast<const uint4*>(qk + (long)(sq.kv_row0 + key) * ldqk + H + h * HD + col);
      rv[cc] = *reinterpret_cast<const uint4*>(vt + (long)(h * HD + r) * ld_vt + sq.vt_col0 + k0 + col);
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
  if (q < sq.q_end) {
    const float inv = 1.0f / l_tot;
    uint16_t* op = out + (long)(sq.out_row0 + q) * ldo + h * HD;
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


// ---------------------------------------------------------------------------
// Split-KV decode attention for the cached solve: <= 32 queries per sequence,
// every query sees all kv_len keys (the active rows' mask row in
// native/model.py:57-75). A workgroup takes DCH keys of one (sequence, head);
// each wave 64 of them, with K and V^T fragments loaded straight from HBM into
// MFMA operand registers (each key is used once, so LDS staging buys nothing).
// The four waves' partial softmax states merge in LDS; chunks merge in
// decode_combine_kernel.
constexpr int DCH = 256;
constexpr int PART = 32 * 66;  // per chunk: m[32], l[32], O[32][64]

__global__ void __launch_bounds__(256)
decode_attention_kernel(const uint16_t* __restrict__ qk, long ldqk, const uint16_t* __restrict__ vt,
                        long ld_vt, const AttnSeq* __restrict__ seqs, int heads, float scale_log2,
                        float* __restrict__ part, int n_chunks) {
  __shared__ float Ow[4][HD][33];
  __shared__ float Mw[4][32], Lw[4][32];
  const AttnSeq sq = seqs[blockIdx.z];
  const int h = blockIdx.y, chunk = blockIdx.x;
  const int kv = sq.kv_len;
  const int k_chunk = chunk * DCH;
  if (k_chunk >= kv) return;  // uniform: nothing of this sequence here
  const int H = heads * HD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nq = sq.q_end - sq.q_begin;

  const int qi = l32 < nq ? l32 : nq - 1;
  bf16x8 qf[4];
  {
    const uint16_t* qp = qk + (long)(sq.q_row0 + sq.q_begin + qi) * ldqk + h * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qp + 16 * kk);
  }
  const int key0 = k_chunk + wave * 64;
  floatx16 s[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
    int key = key0 + kb * 32 + l32;
    key = key < kv ? key : kv - 1;
    const uint16_t* kp = qk + (long)(sq.kv_row0 + key) * ldqk + H + h * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kp + 16 * kk);
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kb], 0, 0, 0);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = key0 + kb * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
      const float sv = key < kv ? s[kb][v] * scale_log2 : -INFINITY;
      s[kb][v] = sv;
      mx = fmaxf(mx, sv);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_safe = mx == -INFINITY ? 0.f : mx;  // a wave entirely past kv_len
  float psum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = exp2f(s[kb][v] - m_safe);
      s[kb][v] = p;
      psum += p;
    }
  psum += __shfl_xor(psum, 32, 64);
  floatx16 o[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[b][v] = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      bf16x8 pf;
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[j] = (__bf16)s[kb][8 * half + j];
      const int kc = key0 + kb * 32 + 16 * half + 4 * hi;  // columns kc..kc+3 and kc+8..kc+11
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const uint16_t* vp = vt + (long)(h * HD + db * 32 + l32) * ld_vt + sq.vt_col0 + kc;
        const uint2 lo = *reinterpret_cast<const uint2*>(vp);
        const uint2 up = *reinterpret_cast<const uint2*>(vp + 8);
        uint4 u = make_uint4(lo.x, lo.y, up.x, up.y);
        const bf16x8 vf = *reinterpret_cast<bf16x8*>(&u);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
      }
    }
  // O^T[d][q] in lanes: q = l32, d = db*32 + 8*(v/4) + 4*hi + v%4
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) Ow[wave][db * 32 + 8 * (v >> 2) + 4 * hi + (v & 3)][l32] = o[db][v];
  if (hi == 0) {
    Mw[wave][l32] = mx;
    Lw[wave][l32] = psum;
  }
  __syncthreads();
  float* pp = part + ((long)(blockIdx.z * heads + h) * n_chunks + chunk) * PART;
  if (tid < 32) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, Mw[w][tid]);
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (Mw[w][tid] != -INFINITY) L += Lw[w][tid] * exp2f(Mw[w][tid] - M);
    pp[tid] = M;
    pp[32 + tid] = L;
  }
  for (int e = tid; e < 32 * HD; e += 256) {
    const int q = e / HD, d = e % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, Mw[w][q]);
    float O = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (Mw[w][q] != -INFINITY) O += Ow[w][d][q] * exp2f(Mw[w][q] - M);
    pp[64 + q * HD + d] = O;
  }
}

__global__ void __launch_bounds__(256)
decode_combine_kernel(const float* __restrict__ part, const AttnSeq* __restrict__ seqs, int heads,
                      int n_chunks, uint16_t* __restrict__ out, long ldo) {
  const AttnSeq sq = seqs[blockIdx.y];
  const int h = blockIdx.x;
  const int nq = sq.q_end - sq.q_begin;
  const int nc = (sq.kv_len + DCH - 1) / DCH;
  const float* pp = part + (long)(blockIdx.y * heads + h) * n_chunks * PART;
  for (int e = threadIdx.x; e < 32 * HD; e += 256) {
    const int q = e / HD, d = e % HD;
    if (q >= nq) continue;
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, pp[c * PART + q]);
    float L = 0.f, O = 0.f;
    for (int c = 0; c < nc; ++c) {
      const float mc = pp[c * PART + q];
      if (mc == -INFINITY) continue;
      const float w = exp2f(mc - M);
      L += pp[c * PART + 32 + q] * w;
      O += pp[c * PART + 64 + q * HD + d] * w;
    }
    out[(long)(sq.out_row0 + sq.q_begin + q) * ldo + h * HD + d] = f2bf(O / L);
  }
}

}  // namespace

hipError_t seq_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                         long ldo, const AttnSeq* seqs, int n_seq, int heads, int max_q, hipStream_t s) {
  if (n_seq <= 0 || max_q <= 0) return hipSuccess;
  const float scale_log2 = 0.125f * 1.4426950408889634f;  // head_dim^-0.5 * log2(e)
  dim3 grid((max_q + BQ - 1) / BQ, heads, n_seq);
  dfh_launch(seq_attention_kernel, grid, dim3(256), 0, s, qk, ldqk, vt, ld_vt, out, ldo, seqs, heads,
             scale_log2);
  return hipGetLastError();
}

hipError_t decode_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                            long ldo, const AttnSeq* seqs, int n_seq, int heads, int max_kv,
                            float* part, hipStream_t s) {
  if (n_seq <= 0 || max_kv <= 0) return hipSuccess;
  const float scale_log2 = 0.125f * 1.4426950408889634f;
  const int n_chunks = (max_kv + DCH - 1) / DCH;
  dfh_launch(decode_attention_kernel, dim3(n_chunks, heads, n_seq), dim3(256), 0, s, qk, ldqk, vt, ld_vt,
             seqs, heads, scale_log2, part, n_chunks);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(heads, n_seq), dim3(256), 0, s, part, seqs, heads, n_chunks,
                     out, ldo);
  return hipGetLastError();
}

}  // namespace dfh
