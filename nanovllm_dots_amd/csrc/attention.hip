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
// Work split: one workgroup = 128 query rows of one (sequence, head); wave w
// owns 32 of them. A work list (one item per existing 128-query tile: the
// sequences with the most tiles first, each sequence's tiles together, longest
// first) is built once per pass; workgroup v takes item v / heads, head
// v % heads, so the dispatcher hands out long tiles early and no workgroup is
// dispatched for a tile that does not exist before all real ones. Workgroup v
// runs on XCD v % 8; with heads a multiple of 8 every query tile of one
// (sequence, head) runs on the same XCD and close in time, so that XCD's L2
// serves their shared K/V tiles.
//
// Per 64-key tile, K and V^T arrive by global->LDS DMA into double-buffered,
// XOR-swizzled tiles (16-B chunk c of row r at slot c ^ ((r >> 1) & 7), which
// keeps the 32-row fragment reads conflict-free). The wave computes
// S^T = K Q^T (32 keys x 32 queries per MFMA block), so a lane holds 32 scores
// of ONE query and the row max needs one cross-lane exchange (lane ^ 32). The
// K rows feeding the MFMA A operand are read with bits 2 and 3 of the row index
// swapped; each lane's accumulators then hold 8 CONSECUTIVE keys per P^T k-step,
// so its V^T operand is one 16-B LDS read. The running max is refreshed only
// when a row's max grows by more than 2^8 (exact: numerator and denominator
// share the stale max; p <= 256 is representable in bf16 and f32), and only
// tiles that cross a row's visible-key limit are masked. exp2 is the hardware
// v_exp_f32 (results below 2^-126 flush to zero: such weights are below one
// f32 ulp of the row's largest weight).
#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

constexpr int BQ = 128;    // query rows per workgroup
constexpr int BKV = 64;    // keys per tile
constexpr int HD = 64;     // head dim
constexpr int NXCD = 8;
constexpr float kRescaleLog2 = 8.0f;  // lazy max refresh threshold (log2 units)

typedef float floatx8 __attribute__((ext_vector_type(8)));

// 64 rows x 128 B tile, swizzled 16-B chunks
__device__ __forceinline__ int att_off(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 7)) << 3); }
// row index with bits 2 and 3 swapped
__device__ __forceinline__ int key_perm(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

// RoPE of a query row held as MFMA B fragments: lane half hi holds dims
// 16*kk + 8*hi + [0, 8) in qf[kk]; the rotation pairs (d, d + 32) are
// (qf[kk], qf[kk + 2]). Factors from the rope_table layout (positions grouped
// by 32: for d = 8g + 4h + t, float ((p/32*4 + g)*64 + p%32*2 + h)*4 + t), so
// one kk needs 8 consecutive floats per table. Same float32 operations as the
// QKV epilogue's RoPE, each result rounded once to bf16.
__device__ __forceinline__ void rope_q(bf16x8 (&qf)[4], int pos, int hi, const float* __restrict__ rope_cos,
                                       const float* __restrict__ rope_sin) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const long o = ((long)((pos >> 5) * 4 + 2 * kk + hi) * 64 + (pos & 31) * 2) * 4;
    const float4 c0 = *reinterpret_cast<const float4*>(rope_cos + o);
    const float4 c1 = *reinterpret_cast<const float4*>(rope_cos + o + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(rope_sin + o);
    const float4 s1 = *reinterpret_cast<const float4*>(rope_sin + o + 4);
    const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x0 = (float)qf[kk][j], x1 = (float)qf[kk + 2][j];
      const float r0 = add_rn(mul_rn(x0, c[j]), mul_rn(-x1, sn[j]));
      const float r1 = add_rn(mul_rn(x1, c[j]), mul_rn(x0, sn[j]));
      qf[kk][j] = (__bf16)r0;
      qf[kk + 2][j] = (__bf16)r1;
    }
  }
}

// One workgroup builds the work list: sequences in order of tile count, most
// first, each sequence's tiles consecutive and longest (highest index) first.
// The dispatcher then hands out the longest tiles early, the shortest last, and
// the query tiles of one (sequence, head) run close together in time, so their
// shared K / V tiles are still in L2. Sequences are bucketed by tile count (the
// last bucket takes every count from kLevels - 1 up); a suffix scan over the
// buckets gives each bucket's first item, and LDS atomics hand out places in a
// bucket.
constexpr int kLevels = 2048;

__global__ void __launch_bounds__(1024) attention_worklist_kernel(const AttnSeq* __restrict__ seqs, int n_seq,
                                                                  char* __restrict__ list) {
  __shared__ int s_start[kLevels];  // items of bucket b, then its next free item
  __shared__ int s_part[1024];
  AttnItem* items = reinterpret_cast<AttnItem*>(list + kAttnListHeader);
  const int tid = threadIdx.x;
  for (int b = tid; b < kLevels; b += 1024) s_start[b] = 0;
  __syncthreads();
  for (int i = tid; i < n_seq; i += 1024) {
    const int L = (seqs[i].q_end - seqs[i].q_begin + BQ - 1) / BQ;
    if (L > 0) atomicAdd(&s_start[min(L, kLevels - 1)], L);
  }
  __syncthreads();
  // exclusive scan from the highest bucket down: thread t owns buckets
  // kLevels-1-2t and kLevels-2-2t
  const int b0 = kLevels - 1 - 2 * tid, b1 = b0 - 1;
  const int a0 = s_start[b0], a1 = s_start[b1];
  s_part[tid] = a0 + a1;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int add = tid >= o ? s_part[tid - o] : 0;
    __syncthreads();
    s_part[tid] += add;
    __syncthreads();
  }
  const int excl = s_part[tid] - (a0 + a1);
  s_start[b0] = excl;
  s_start[b1] = excl + a0;
  __syncthreads();
  for (int i = tid; i < n_seq; i += 1024) {
    const AttnSeq sq = seqs[i];
    const int L = (sq.q_end - sq.q_begin + BQ - 1) / BQ;
    if (L <= 0) continue;
    const int off = atomicAdd(&s_start[min(L, kLevels - 1)], L);
    for (int k = 0; k < L; ++k) {
      AttnItem it;
      it.seq = sq;
      it.tile = L - 1 - k;
#pragma unroll
      for (int q = 0; q < 7; ++q) it.pad[q] = 0;
      items[off + k] = it;
    }
  }
  if (tid == 0) *reinterpret_cast<int*>(list) = s_part[1023];
}

__global__ void __launch_bounds__(256, 3)
seq_attention_kernel(const uint16_t* __restrict__ qk, long ldqk, const uint16_t* __restrict__ vt,
                     long ld_vt, uint16_t* __restrict__ out, long ldo, int heads,
                     const char* __restrict__ list, float scale_log2, const float* __restrict__ rope_cos,
                     const float* __restrict__ rope_sin) {
  __shared__ __attribute__((aligned(16))) uint16_t K0[BKV * HD];
  __shared__ __attribute__((aligned(16))) uint16_t K1[BKV * HD];
  __shared__ __attribute__((aligned(16))) uint16_t V0[HD * BKV];
  __shared__ __attribute__((aligned(16))) uint16_t V1[HD * BKV];

  const int v = blockIdx.x;
  if (v >= *reinterpret_cast<const int*>(list) * heads) return;
  const AttnItem item = reinterpret_cast<const AttnItem*>(list + kAttnListHeader)[v / heads];
  const int h = v % heads;
  const AttnSeq sq = item.seq;
  const int q0 = sq.q_begin + item.tile * BQ;
  const int T = sq.kv_len;           // keys of full rows
  const int cend = sq.causal_end;    // queries below this are causal
  const int H = heads * HD;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;

  // visible keys of query q: [0, q+1) below cend, [0, T) from cend on (monotone in q)
  auto limit = [&](int q) { return q < cend ? q + 1 : T; };
  const int kmax = limit(min(q0 + BQ, sq.q_end) - 1);  // keys this workgroup needs
  const int ntiles = (kmax + BKV - 1) / BKV;

  const int q = q0 + wave * 32 + l32;
  const int qc = q < sq.q_end ? q : sq.q_end - 1;
  const int lim = limit(qc);
  const int wq_first = q0 + wave * 32;
  const bool wave_on = wq_first < sq.q_end;
  const int wave_kmax = wave_on ? limit(min(wq_first + 31, sq.q_end - 1)) : 0;  // keys any lane sees
  const int wave_kall = wave_on ? limit(wq_first) : 0;                          // keys every lane sees

  // Q fragments (B operand): Q[q][16*kk + 8*hi .. +8]
  bf16x8 qf[4];
  {
    const uint16_t* qp = qk + (long)(sq.q_row0 + qc) * ldqk + h * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qp + 16 * kk);
  }
  if (rope_cos) rope_q(qf, qc, hi, rope_cos, rope_sin);  // uniform

  // DMA: wave w, load j covers tile rows [(4j + w) * 8, +8); lane -> row + lane/8, slot lane%8
  const int dma_r0 = wave * 8 + (lane >> 3);
  const int dma_c = lane & 7;
  const uint16_t* kbase = qk + (long)sq.kv_row0 * ldqk + H + h * HD;
  const uint16_t* vbase = vt + (long)(h * HD) * ld_vt + sq.vt_col0;
  auto dma = [&](uint16_t* kd, uint16_t* vd, int k0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = j * 32 + dma_r0;
      const int c = dma_c ^ ((r >> 1) & 7);
      const int key = min(k0 + r, T - 1);
      __builtin_amdgcn_global_load_lds(DFH_GPTR(kbase + (long)key * ldqk + c * 8),
                                       DFH_LPTR(kd + (j * 32 + wave * 8) * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(DFH_GPTR(vbase + (long)r * ld_vt + k0 + c * 8),
                                       DFH_LPTR(vd + (j * 32 + wave * 8) * 64), 16, 0, 0);
    }
  };

  floatx16 o[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[b][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float thr = kRescaleLog2 / scale_log2;  // in raw score units
  const int krow = key_perm(l32);

  auto compute = [&](const uint16_t* Ks, const uint16_t* Vs, int k0) {
    if (k0 >= wave_kmax) return;  // wave-uniform
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(Ks + att_off(kb * 32 + krow, 2 * kk + hi));
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kb], 0, 0, 0);
      }
    }
    // accumulator v of block kb holds key k0 + kb*32 + 16*(v/8) + 8*hi + v%8
    if (k0 + BKV > wave_kall) {
      const int rel = lim - k0 - 8 * hi;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (kb * 32 + 16 * (v >> 3) + (v & 7) >= rel) s[kb][v] = -INFINITY;
    }
    float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int v = 2; v < 16; ++v) mx = fmaxf(mx, s[0][v]);
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[1][v]);
    mx = fmaxf(mx, swap_halves(mx));
    if (__any(mx > m_run + thr)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[b][v] *= alpha;
    }
    const float mb = m_run * scale_log2;
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][v], scale_log2, -mb));
        s[kb][v] = p;
        psum += p;
      }
    l_run += psum;
    // O^T[d][q] += V^T[d][keys] P^T[keys][q]; k-step (kb, half) = keys kb*32 + 16*half + [0, 16)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        floatx8 pv;
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = s[kb][8 * half + j];
        const bf16x8 pf = __builtin_convertvector(pv, bf16x8);
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 vf =
              *reinterpret_cast<const bf16x8*>(Vs + att_off(db * 32 + l32, 4 * kb + 2 * half + hi));
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
        }
      }
  };

  dma(K0, V0, 0);
  for (int t = 0; t < ntiles; t += 2) {
    wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    if (t + 1 < ntiles) dma(K1, V1, (t + 1) * BKV);
    compute(K0, V0, t * BKV);
    if (t + 1 >= ntiles) break;
    wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    if (t + 2 < ntiles) dma(K0, V0, (t + 2) * BKV);
    compute(K1, V1, (t + 1) * BKV);
  }

  const float l_tot = l_run + swap_halves(l_run);
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
// each wave 64 of them. Each key is used once, so a wave stages only its own
// 64-key K and V^T tiles: global->LDS DMA moves whole 128-B lines (8 lines per
// 1 KB instruction), where direct operand loads would touch 32 lines per
// instruction and every V^T line eight times. The tiles use the swizzle and
// the key-row permutation of seq_attention_kernel. The four waves' partial
// softmax states merge in LDS (over the tiles' space); chunks merge in
// decode_combine_kernel.
constexpr int DCH = 256;
constexpr int PART = 32 * 66;  // per chunk: m[32], l[32], O[32][64]

__global__ void __launch_bounds__(256)
decode_attention_kernel(const uint16_t* __restrict__ qk, long ldqk, const uint16_t* __restrict__ vt,
                        long ld_vt, const AttnSeq* __restrict__ seqs, int heads, float scale_log2,
                        float* __restrict__ part, int n_chunks, const float* __restrict__ rope_cos,
                        const float* __restrict__ rope_sin) {
  // per wave: K tile [64 keys][64] then V^T tile [64 d][64 keys], 16 KB; after the
  // scores and P.V the same space holds the waves' O^T for the merge
  __shared__ __attribute__((aligned(16))) uint16_t tiles[4 * 2 * BKV * HD];
  __shared__ float Mw[4][32], Lw[4][32];
  float (*Ow)[HD][33] = reinterpret_cast<float (*)[HD][33]>(tiles);
  static_assert(sizeof(float) * 4 * HD * 33 <= sizeof(uint16_t) * 4 * 2 * BKV * HD, "merge space");
  const AttnSeq sq = seqs[blockIdx.z];
  const int h = blockIdx.y, chunk = blockIdx.x;
  const int kv = sq.kv_len;
  const int k_chunk = chunk * DCH;
  if (k_chunk >= kv) return;  // uniform: nothing of this sequence here
  const int H = heads * HD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nq = sq.q_end - sq.q_begin;
  const int key0 = k_chunk + wave * BKV;
  uint16_t* Kw = tiles + wave * 2 * BKV * HD;
  uint16_t* Vw = Kw + BKV * HD;
  // DMA: load j fills tile rows [8j, 8j + 8): lane -> row 8j + lane/8, slot lane%8,
  // which holds source chunk (lane%8) ^ swz(row). K rows past kv_len repeat the
  // last key (masked below); V^T columns past it are finite (zeroed slack)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = j * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int key = min(key0 + r, kv - 1);
    __builtin_amdgcn_global_load_lds(DFH_GPTR(qk + (long)(sq.kv_row0 + key) * ldqk + H + h * HD + c * 8),
                                     DFH_LPTR(Kw + j * 8 * HD), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(DFH_GPTR(vt + (long)(h * HD + r) * ld_vt + sq.vt_col0 + key0 + c * 8),
                                     DFH_LPTR(Vw + j * 8 * BKV), 16, 0, 0);
  }
  const int qi = l32 < nq ? l32 : nq - 1;
  bf16x8 qf[4];
  {
    const uint16_t* qp = qk + (long)(sq.q_row0 + sq.q_begin + qi) * ldqk + h * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qp + 16 * kk);
  }
  if (rope_cos) rope_q(qf, sq.q_begin + qi, hi, rope_cos, rope_sin);  // uniform
  wait_vm_lgkm0<0>();  // this wave's tiles are in LDS (only this wave reads them)
  const int krow = key_perm(l32);
  floatx16 s[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(Kw + att_off(kb * 32 + krow, 2 * kk + hi));
      s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kb], 0, 0, 0);
    }
  }
  // accumulator v of block kb holds key key0 + kb*32 + 16*(v/8) + 8*hi + v%8
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = key0 + kb * 32 + 16 * (v >> 3) + 8 * hi + (v & 7);
      const float sv = key < kv ? s[kb][v] * scale_log2 : -INFINITY;
      s[kb][v] = sv;
      mx = fmaxf(mx, sv);
    }
  mx = fmaxf(mx, swap_halves(mx));
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
  psum += swap_halves(psum);
  floatx16 o[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[b][v] = 0.f;
  // O^T[d][q] += V^T[d][keys] P^T[keys][q]; k-step (kb, half) = keys kb*32 + 16*half + [0, 16)
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      floatx8 pv;
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = s[kb][8 * half + j];
      const bf16x8 pf = __builtin_convertvector(pv, bf16x8);
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(Vw + att_off(db * 32 + l32, 4 * kb + 2 * half + hi));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
      }
    }
  __syncthreads();  // every wave is done with its tiles: their space becomes Ow
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

// Merge of the chunk partials: one workgroup per (sequence, head, group of
// DQG queries). Per block of up to DCB chunks, the chunk weights
// exp2(m_c - M) / L of the group's queries go to LDS; then every thread adds
// two output columns of one query over the block's chunks with independent
// loads (64 threads per query read its 256-B O rows coalesced).
constexpr int DQG = 8;    // queries per combine workgroup
constexpr int DCB = 256;  // chunks per LDS block of weights

__global__ void __launch_bounds__(256)
decode_combine_kernel(const float* __restrict__ part, const AttnSeq* __restrict__ seqs, int heads,
                      int n_chunks, uint16_t* __restrict__ out, long ldo) {
  __shared__ float Ws[DQG][DCB];
  __shared__ float Mq[DQG], Lq[DQG];
  const AttnSeq sq = seqs[blockIdx.y];
  const int h = blockIdx.x, qg = blockIdx.z * DQG;
  const int nq = sq.q_end - sq.q_begin;
  if (qg >= nq) return;  // uniform
  const int R = min(DQG, nq - qg);
  const int nc = min((sq.kv_len + DCH - 1) / DCH, n_chunks);
  const float* pp = part + (long)(blockIdx.y * heads + h) * n_chunks * PART;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // row max and sum of each query over all chunks: wave w takes queries w and w + 4
  for (int r = wave; r < R; r += 4) {
    const int q = qg + r;
    float M = -INFINITY;
    for (int c = lane; c < nc; c += 64) M = fmaxf(M, pp[(long)c * PART + q]);
    M = wave_max(M);
    float L = 0.f;
    if (M != -INFINITY)
      for (int c = lane; c < nc; c += 64) {
        const float mc = pp[(long)c * PART + q];
        if (mc != -INFINITY) L += pp[(long)c * PART + 32 + q] * exp2f(mc - M);
      }
    L = wave_sum(L);
    if (lane == 0) { Mq[r] = M; Lq[r] = L; }
  }
  __syncthreads();
  const int r = tid >> 5, d = (tid & 31) * 2;  // this thread's query and two output columns
  float o0 = 0.f, o1 = 0.f;
  for (int c0 = 0; c0 < nc; c0 += DCB) {
    const int cn = min(DCB, nc - c0);
    for (int idx = tid; idx < R * cn; idx += 256) {
      const int rr = idx / cn, cc = idx % cn;
      const float mc = pp[(long)(c0 + cc) * PART + qg + rr];
      const float M = Mq[rr], L = Lq[rr];
      Ws[rr][cc] = (L > 0.f && mc != -INFINITY) ? exp2f(mc - M) / L : 0.f;
    }
    __syncthreads();
    if (r < R) {
      const float* po = pp + (long)c0 * PART + 64 + (qg + r) * HD + d;
#pragma unroll 8
      for (int cc = 0; cc < cn; ++cc) {
        const float w = Ws[r][cc];
        const float2 x = *reinterpret_cast<const float2*>(po + (long)cc * PART);
        o0 += w != 0.f ? w * x.x : 0.f;
        o1 += w != 0.f ? w * x.y : 0.f;
      }
    }
    __syncthreads();
  }
  if (r < R)
    *reinterpret_cast<uint32_t*>(out + (long)(sq.out_row0 + sq.q_begin + qg + r) * ldo + h * HD + d) =
        pack2(o0, o1);
}

}  // namespace

hipError_t attention_worklist(const AttnSeq* seqs, int n_seq, void* list, hipStream_t s) {
  if (n_seq < 0 || n_seq >= (1 << 24)) return hipErrorInvalidValue;
  dfh_launch(attention_worklist_kernel, dim3(1), dim3(1024), 0, s, seqs, n_seq, reinterpret_cast<char*>(list));
  return hipGetLastError();
}

hipError_t seq_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                         long ldo, int heads, const void* list, long max_items, const float* rope_cos,
                         const float* rope_sin, hipStream_t s) {
  if (max_items <= 0) return hipSuccess;
  const float scale_log2 = 0.125f * 1.4426950408889634f;  // head_dim^-0.5 * log2(e)
  const long grid = max_items * heads;
  if (grid > 0x7fffffffL) return hipErrorInvalidValue;
  dfh_launch(seq_attention_kernel, dim3((unsigned)grid), dim3(256), 0, s, qk, ldqk, vt, ld_vt, out, ldo, heads,
             reinterpret_cast<const char*>(list), scale_log2, rope_cos, rope_sin);
  return hipGetLastError();
}

hipError_t decode_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                            long ldo, const AttnSeq* seqs, int n_seq, int heads, int max_kv,
                            float* part, const float* rope_cos, const float* rope_sin, hipStream_t s) {
  if (n_seq <= 0 || max_kv <= 0) return hipSuccess;
  const float scale_log2 = 0.125f * 1.4426950408889634f;
  const int n_chunks = (max_kv + DCH - 1) / DCH;
  dfh_launch(decode_attention_kernel, dim3(n_chunks, heads, n_seq), dim3(256), 0, s, qk, ldqk, vt, ld_vt,
             seqs, heads, scale_log2, part, n_chunks, rope_cos, rope_sin);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(heads, n_seq, 32 / DQG), dim3(256), 0, s, part, seqs, heads,
                     n_chunks, out, ldo);
  return hipGetLastError();
}

}  // namespace dfh
