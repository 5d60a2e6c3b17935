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
#include <algorithm>
#include <type_traits>

#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

constexpr int BQ = 128;    // query rows per workgroup
constexpr int BKV = 64;    // keys per tile
constexpr int HD = 64;     // head dim
constexpr int NXCD = 8;
constexpr float kRescaleLog2 = 8.0f;  // lazy max refresh threshold (log2 units)
// buffer resource word 3 for gfx9-family raw (stride 0) buffers: 32-bit data format
constexpr int kBufferFlags = 0x00020000;

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

  // DMA: wave w, load j covers tile rows [(4j + w) * 8, +8); lane -> row + lane/8, slot lane%8.
  // Buffer loads: a lane's byte offsets are the same for every tile. K rows
  // through a resource that starts at the tile's first key and ends at key
  // min(T, first key + 64): rows past the sequence arrive as zeros (their
  // scores are masked). V^T columns at the tile's key offset (soffset);
  // columns past T are read as they are (finite; their weights are zero). The
  // launcher keeps every byte offset below 2^31.
  const int dma_r0 = wave * 8 + (lane >> 3);
  const int dma_c = lane & 7;
  const uint16_t* kbase = qk + (long)sq.kv_row0 * ldqk + H + h * HD;
  uint32_t koff[2], voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = j * 32 + dma_r0;
    const int c = dma_c ^ ((r >> 1) & 7);
    koff[j] = ((uint32_t)r * (uint32_t)ldqk + (uint32_t)c * 8u) * 2u;
    voff[j] = ((uint32_t)r * (uint32_t)ld_vt + (uint32_t)c * 8u) * 2u;
  }
  const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(vt + (long)(h * HD) * ld_vt + sq.vt_col0), (short)0, (int)((uint32_t)HD * (uint32_t)ld_vt * 2u),
      kBufferFlags);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // the LDS destinations (M0) in scalars
  auto dma = [&](uint16_t* kd, uint16_t* vd, int k0) {
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kbase + (long)k0 * ldqk), (short)0, (int)((uint32_t)min(T - k0, BKV) * (uint32_t)ldqk * 2u),
        kBufferFlags);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kres, DFH_LPTR(kd + (j * 32 + wave_u * 8) * 64), 16, koff[j], 0, 0,
                                               0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vres, DFH_LPTR(vd + (j * 32 + wave_u * 8) * 64), 16, voff[j], k0 * 2,
                                               0, 0);
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
  // per-lane byte offsets of the fragment reads within a stage (a tile's
  // second 32-row block starts 4096 B on, with the same swizzle)
  uint32_t krd[4], vrd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) krd[kk] = (uint32_t)att_off(krow, 2 * kk + hi) * 2u;
#pragma unroll
  for (int c = 0; c < 4; ++c) vrd[c] = (uint32_t)att_off(l32, 2 * c + hi) * 2u;  // k-step (kb, half): c = 2kb + half

  // one 16-B fragment read per (lane address, block): the stage's base is added
  // once per address, the block offset rides in the instruction
  auto frag = [](uint32_t addr, int off) {
    return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>((uintptr_t)(addr + off));
  };
  // masked: the tile crosses some lane's visible-key limit (wave-uniform test
  // at the call site; two copies of the tile code, so unmasked tiles carry no
  // per-score compare and select)
  auto compute = [&](auto masked, const uint16_t* Ks, const uint16_t* Vs, int k0) {
    const uint32_t kst = (uint32_t)(uintptr_t)DFH_LPTR(Ks), vst = (uint32_t)(uintptr_t)DFH_LPTR(Vs);
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint32_t ka = kst + krd[kk];
      asm volatile("" : "+v"(ka));  // keeps the block offset out of the address sum
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(ka, kb * 4096), qf[kk], s[kb], 0, 0, 0);
    }
    // accumulator v of block kb holds key k0 + kb*32 + 16*(v/8) + 8*hi + v%8
    if constexpr (decltype(masked)::value) {
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
        uint32_t va = vst + vrd[2 * kb + half];
        asm volatile("" : "+v"(va));
#pragma unroll
        for (int db = 0; db < 2; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(va, db * 4096), pf, o[db], 0, 0, 0);
      }
  };

  auto tile = [&](const uint16_t* Ks, const uint16_t* Vs, int k0) {
    if (k0 >= wave_kmax) return;  // wave-uniform: no key of the tile is visible to the wave
    if (k0 + BKV > wave_kall) compute(std::true_type{}, Ks, Vs, k0);
    else compute(std::false_type{}, Ks, Vs, k0);
  };
  // one tile per iteration (stage t % 2): a single copy of the tile code keeps
  // the kernel at 123 VGPRs, four workgroups per CU
  dma(K0, V0, 0);
  for (int t = 0; t < ntiles; ++t) {
    wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    const bool odd = t & 1;
    if (t + 1 < ntiles) dma(odd ? K0 : K1, odd ? V0 : V1, (t + 1) * BKV);
    tile(odd ? K1 : K0, odd ? V1 : V0, t * BKV);
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
// native/model.py:57-75). Group g = (sequence, head) is cut into chunks of
// chunk_keys consecutive keys, one workgroup each, about one workgroup per CU
// in all. Wave w of a chunk's workgroup takes the chunk's 64-key tiles
// w, w + NWV, ...: it stages each tile's K rows and V^T columns in its own LDS
// by global->LDS DMA (whole 128-B lines, the swizzle and key-row permutation of
// seq_attention_kernel) and scores it with the online softmax of
// seq_attention_kernel (lazy max refresh); the next tile streams in while this
// one is scored (a second stage, or the other wave of the SIMD). Only the wave
// reads its tiles: no barrier inside the key loop. Only the sequence's last
// tile is masked. The waves' softmax states merge in LDS. A group of one chunk
// writes its rows there; otherwise each chunk stores its partial (m in log2
// units, l, O of its <= 32 queries) and the last chunk of the group to finish
// merges the group's partials (one round of loads for up to 8 chunks) and
// writes the rows. The chunks of a group are dealt to workgroups with one
// value of blockIdx.x % 8, which the 8-XCD partition mode places on one XCD:
// their partials meet in that XCD's L2. A chunk that finds itself on another
// XCD (hardware register XCC_ID) publishes with an
// agent-scope release fence and marks the group's counter, and the merging
// chunk of a marked group takes an agent-scope acquire fence. The last arriver
// zeroes the counter for the next launch.
constexpr int PART = 32 * 66;         // per chunk: m[32], l[32], O[32][64]
constexpr int kDecodeMaxChunks = 64;  // chunks per group (merge weights in LDS)
constexpr int kWaveTile = 2 * BKV * HD;  // K tile then V^T tile, uint16_t elements
// NWV waves per workgroup, NST stages per wave (tiles in flight per wave: NST - 1).
// 8 waves of one stage (two waves per SIMD, 128 KB of tiles): while one wave of
// a SIMD waits for its next tile the other computes.
constexpr int kDecodeWaves = 8, kDecodeStages = 1;

template <int NWV, int NST>
__global__ void __launch_bounds__(64 * NWV)
decode_attention_kernel(const uint16_t* __restrict__ qk, long ldqk, const uint16_t* __restrict__ vt,
                        long ld_vt, const AttnSeq* __restrict__ seqs, int heads, int n_groups, int n_chunks,
                        int chunk_keys, float scale_log2, float* __restrict__ part, unsigned* __restrict__ cnt,
                        uint16_t* __restrict__ out, long ldo, const float* __restrict__ rope_cos,
                        const float* __restrict__ rope_sin) {
  // per wave NST stages of (K tile [64 keys][64], V^T tile [64 d][64 keys]), 16 KB
  // each; after the key loop the wave's first 8.4 KB hold its O^T for the merge
  constexpr int DWV = NWV, NT = 64 * NWV;
  static_assert(NST >= 1 && NST <= 4, "stages");
  __shared__ __attribute__((aligned(16))) uint16_t tiles[DWV * NST * kWaveTile];
  __shared__ float Mw[DWV][32], Lw[DWV][32];
  __shared__ float Ws[kDecodeMaxChunks][32];
  __shared__ int s_flag;
  const int xcd = blockIdx.x % NXCD, j = blockIdx.x / NXCD;
  const int g = xcd + NXCD * (j / n_chunks), chunk = j % n_chunks;
  if (g >= n_groups) return;  // uniform: padding of the group count to a multiple of 8
  const int si = g / heads, h = g % heads;
  const AttnSeq sq = seqs[si];
  const int kv = sq.kv_len;
  const int k_lo = chunk * chunk_keys;
  if (k_lo >= kv) return;  // uniform: nothing of this sequence here (not counted below)
  const int k_hi = min(k_lo + chunk_keys, kv);
  const int nc = min((kv + chunk_keys - 1) / chunk_keys, n_chunks);  // chunks of this group
  const int H = heads * HD;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: tile and LDS bases in SGPRs
  const int l32 = lane & 31, hi = lane >> 5;
  const int nq = sq.q_end - sq.q_begin;
  const int n_t = (k_hi - k_lo + BKV - 1) / BKV;                 // tiles of the chunk
  const int nw = n_t > wave ? (n_t - wave + DWV - 1) / DWV : 0;  // this wave's tiles
  uint16_t* st0 = tiles + wave * NST * kWaveTile;
  const uint16_t* kbase = qk + (long)sq.kv_row0 * ldqk + H + h * HD;
  const uint16_t* vbase = vt + (long)(h * HD) * ld_vt + sq.vt_col0;
  // DMA of the wave's tile i (keys k_lo + (wave + 4i) * 64 + [0, 64)) into a stage:
  // load j fills tile rows [8j, 8j + 8): lane -> row 8j + lane/8, slot lane%8,
  // which holds source chunk (lane%8) ^ swz(row); swz(row) = ((row >> 1) & 7)
  // takes one value per lane for even j and another for odd j. Addresses are a
  // uniform base per (tile, j) plus a per-lane byte offset that never changes.
  // Tiles start at multiples of 64 keys of the sequence, and the caller's key
  // space (a cache region) comes in whole 64-key tiles: rows and columns past
  // kv_len stay inside it and hold finite values (K scores there are masked,
  // their P is zero).
  const uint32_t lr = lane >> 3;
  const uint32_t k_off0 = (lr * (uint32_t)ldqk + (uint32_t)(((lane & 7) ^ ((lr >> 1) & 7)) * 8)) * 2u;
  const uint32_t k_off1 = (lr * (uint32_t)ldqk + (uint32_t)(((lane & 7) ^ (((lr >> 1) + 4) & 7)) * 8)) * 2u;
  const uint32_t v_off0 = (lr * (uint32_t)ld_vt + (uint32_t)(((lane & 7) ^ ((lr >> 1) & 7)) * 8)) * 2u;
  const uint32_t v_off1 = (lr * (uint32_t)ld_vt + (uint32_t)(((lane & 7) ^ (((lr >> 1) + 4) & 7)) * 8)) * 2u;
  auto dma = [&](uint16_t* stage, int i) {
    const int key0 = k_lo + (wave + DWV * i) * BKV;
    const char* kt = reinterpret_cast<const char*>(kbase + (long)key0 * ldqk);
    const char* vtt = reinterpret_cast<const char*>(vbase + key0);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const char* kj = kt + (long)jj * 8 * ldqk * 2;
      const char* vj = vtt + (long)jj * 8 * ld_vt * 2;
      __builtin_amdgcn_global_load_lds(DFH_GPTR(kj + ((jj & 1) ? k_off1 : k_off0)),
                                       DFH_LPTR(stage + jj * 8 * HD), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(DFH_GPTR(vj + ((jj & 1) ? v_off1 : v_off0)),
                                       DFH_LPTR(stage + BKV * HD + jj * 8 * BKV), 16, 0, 0);
    }
  };
  if (nw > 0) dma(st0, 0);
  const int qi = l32 < nq ? l32 : nq - 1;
  bf16x8 qf[4];
  {
    const uint16_t* qp = qk + (long)(sq.q_row0 + sq.q_begin + qi) * ldqk + h * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qp + 16 * kk);
  }
  if (rope_cos) rope_q(qf, sq.q_begin + qi, hi, rope_cos, rope_sin);  // uniform
  const int krow = key_perm(l32);
  floatx16 o[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[b][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float thr = kRescaleLog2 / scale_log2;  // in raw score units

  auto compute = [&](auto masked, const uint16_t* Ks, const uint16_t* Vs, int k0) {
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
    if constexpr (decltype(masked)::value) {  // the sequence's last tile
      const int rel = kv - k0 - 8 * hi;
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
    mx = fmaxf(mx, swap_halves(mx));  // finite: every tile holds a key below kv_len
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
        for (int jv = 0; jv < 8; ++jv) pv[jv] = s[kb][8 * half + jv];
        const bf16x8 pf = __builtin_convertvector(pv, bf16x8);
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 vf =
              *reinterpret_cast<const bf16x8*>(Vs + att_off(db * 32 + l32, 4 * kb + 2 * half + hi));
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
        }
      }
  };

  // Tile i sits in stage i % NST; tiles 0 .. NST - 2 go out first. At the top of
  // step i the wave waits for tile i (the tiles after it, at most NST - 2 of
  // them, may stay in flight: 16 DMA instructions each, completing in order) and
  // for its LDS reads of tile i - 1, then starts tile i + NST - 1 into the stage
  // tile i - 1 used. One stage: tile i + 1 starts once tile i's LDS reads are
  // done, and the other waves of the SIMD compute meanwhile.
  for (int i = 1; i < NST - 1 && i < nw; ++i) dma(st0 + i * kWaveTile, i);
  for (int i = 0, si = 0; i < nw; ++i, si = si + 1 == NST ? 0 : si + 1) {
    const int ahead = min(NST - 2, nw - 1 - i);
    if (ahead <= 0) wait_vm_lgkm0<0>();
    else if (ahead == 1) wait_vm_lgkm0<16>();
    else wait_vm_lgkm0<32>();
    if (NST > 1 && i + NST - 1 < nw) dma(st0 + (si == 0 ? NST - 1 : si - 1) * kWaveTile, i + NST - 1);
    uint16_t* sb = st0 + si * kWaveTile;
    const int k0 = k_lo + (wave + DWV * i) * BKV;
    if (k0 + BKV <= kv) compute(std::false_type{}, sb, sb + BKV * HD, k0);
    else compute(std::true_type{}, sb, sb + BKV * HD, k0);
    if (NST == 1 && i + 1 < nw) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the tile's LDS reads are done
      dma(st0, i + 1);
    }
  }
  wait_vm_lgkm0<0>();  // (a wave without tiles) nothing outstanding into its stages
  // O^T[d][q] in lanes: q = l32, d = db*32 + 8*(v/4) + 4*hi + v%4; the wave's own stage space
  float (*Ow)[33] = reinterpret_cast<float (*)[33]>(st0);
  static_assert(sizeof(float) * HD * 33 <= sizeof(uint16_t) * NST * kWaveTile, "merge space");
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) Ow[db * 32 + 8 * (v >> 2) + 4 * hi + (v & 3)][l32] = o[db][v];
  const float l_tot = l_run + swap_halves(l_run);
  if (hi == 0) {
    Mw[wave][l32] = nw > 0 ? m_run * scale_log2 : -INFINITY;
    Lw[wave][l32] = l_tot;
  }
  __syncthreads();
  auto ow = [&](int w) { return reinterpret_cast<const float (*)[33]>(tiles + w * NST * kWaveTile); };
  // merge of the four waves for query q: max M, weight of wave w = exp2(m_w - M)
  auto wave_merge = [&](int q, float& M, float (&wt)[DWV]) {
    M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DWV; ++w) M = fmaxf(M, Mw[w][q]);
#pragma unroll
    for (int w = 0; w < DWV; ++w) wt[w] = Mw[w][q] != -INFINITY ? __builtin_amdgcn_exp2f(Mw[w][q] - M) : 0.f;
  };
  if (nc == 1) {  // the group's only chunk: normalised rows straight out
    for (int e = tid; e < nq * (HD / 2); e += NT) {
      const int q = e / (HD / 2), d = 2 * (e % (HD / 2));
      float M, wt[DWV];
      wave_merge(q, M, wt);
      float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
      for (int w = 0; w < DWV; ++w) {
        L += Lw[w][q] * wt[w];
        o0 += ow(w)[d][q] * wt[w];
        o1 += ow(w)[d + 1][q] * wt[w];
      }
      const float inv = 1.0f / L;
      *reinterpret_cast<uint32_t*>(out + (long)(sq.out_row0 + sq.q_begin + q) * ldo + h * HD + d) =
          pack2(o0 * inv, o1 * inv);
    }
    return;
  }
  float* pg = part + (long)g * n_chunks * PART;  // the group's partials
  {
    float* pp = pg + (long)chunk * PART;
    if (tid < nq) {
      float M, wt[DWV];
      wave_merge(tid, M, wt);
      float L = 0.f;
#pragma unroll
      for (int w = 0; w < DWV; ++w) L += Lw[w][tid] * wt[w];
      pp[tid] = M;
      pp[32 + tid] = L;
    }
    for (int e = tid; e < nq * HD; e += NT) {
      const int q = e / HD, d = e % HD;
      float M, wt[DWV];
      wave_merge(q, M, wt);
      float O = 0.f;
#pragma unroll
      for (int w = 0; w < DWV; ++w) O += ow(w)[d][q] * wt[w];
      pp[64 + q * HD + d] = O;
    }
  }
  const bool on_xcd = __builtin_amdgcn_s_getreg((3 << 11) | 20) == xcd;  // hwreg(XCC_ID, 0, 4); uniform
  if (!on_xcd) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial stores are in L2
  __syncthreads();                                   // ... and every wave's
  if (tid == 0) {
    const unsigned add = on_xcd ? 1u : 0x10001u;
    const unsigned now = __hip_atomic_fetch_add(cnt + g, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
    s_flag = (now & 0xffffu) != (unsigned)nc ? 0 : (now >> 16) ? 2 : 1;
  }
  __syncthreads();
  if (!s_flag) return;  // uniform
  if (s_flag == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  asm volatile("" ::: "memory");
  if (tid == 0) cnt[g] = 0u;  // ready for the next launch
  // Last chunk in. Up to CB chunks: each thread loads m, l and its two O columns
  // of every chunk at once (one round trip; the 32 threads of a query share the
  // m / l addresses), then M = max m_c, L = sum l_c exp2(m_c - M) and
  // O = sum exp2(m_c - M) / L * O_c, each in chunk order. More chunks: the chunk
  // weights go through LDS first.
  constexpr int CB = 8;
  if (nc <= CB) {
    for (int e = tid; e < nq * (HD / 2); e += NT) {
      const int q = e / (HD / 2), d = 2 * (e % (HD / 2));
      float mc[CB], lc[CB];
      float2 x[CB];
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        const float* pc = pg + (long)min(b, nc - 1) * PART;
        mc[b] = pc[q];
        lc[b] = pc[32 + q];
        x[b] = *reinterpret_cast<const float2*>(pc + 64 + q * HD + d);
      }
      float M = -INFINITY;
#pragma unroll
      for (int b = 0; b < CB; ++b)
        if (b < nc) M = fmaxf(M, mc[b]);
      float L = 0.f;
#pragma unroll
      for (int b = 0; b < CB; ++b)
        if (b < nc && mc[b] != -INFINITY) L += lc[b] * __builtin_amdgcn_exp2f(mc[b] - M);
      const float inv = 1.0f / L;
      float o0 = 0.f, o1 = 0.f;
#pragma unroll
      for (int b = 0; b < CB; ++b)
        if (b < nc) {
          const float w = mc[b] != -INFINITY ? __builtin_amdgcn_exp2f(mc[b] - M) * inv : 0.f;
          o0 += w * x[b].x;
          o1 += w * x[b].y;
        }
      *reinterpret_cast<uint32_t*>(out + (long)(sq.out_row0 + sq.q_begin + q) * ldo + h * HD + d) = pack2(o0, o1);
    }
    return;
  }
  // every chunk's m and l to LDS (one load per thread and pair; Ow is dead: the
  // second stage of wave 0), per query the chunk weights, then the O columns
  // over the chunks in chunk order, CB chunks' loads in flight together
  float (*Mc)[32] = reinterpret_cast<float (*)[32]>(tiles + kWaveTile);
  float (*Lc)[32] = Mc + kDecodeMaxChunks;
  static_assert(2 * kDecodeMaxChunks * 32 * sizeof(float) <= kWaveTile * sizeof(uint16_t), "m / l space");
  for (int e = tid; e < nc * 32; e += NT) {
    const int c = e >> 5, q = e & 31;
    Mc[c][q] = pg[(long)c * PART + q];
    Lc[c][q] = pg[(long)c * PART + 32 + q];
  }
  __syncthreads();
  if (tid < nq) {
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, Mc[c][tid]);
    float L = 0.f;
    for (int c = 0; c < nc; ++c) {
      const float mc = Mc[c][tid];
      if (mc != -INFINITY) L += Lc[c][tid] * __builtin_amdgcn_exp2f(mc - M);
    }
    const float inv = 1.0f / L;
    for (int c = 0; c < nc; ++c) {
      const float mc = Mc[c][tid];
      Ws[c][tid] = mc != -INFINITY ? __builtin_amdgcn_exp2f(mc - M) * inv : 0.f;
    }
  }
  __syncthreads();
  for (int e = tid; e < nq * (HD / 2); e += NT) {
    const int q = e / (HD / 2), d = 2 * (e % (HD / 2));
    const float* po = pg + 64 + q * HD + d;
    float o0 = 0.f, o1 = 0.f;
    for (int c0 = 0; c0 < nc; c0 += CB) {
      float2 x[CB];
#pragma unroll
      for (int b = 0; b < CB; ++b) x[b] = *reinterpret_cast<const float2*>(po + (long)min(c0 + b, nc - 1) * PART);
#pragma unroll
      for (int b = 0; b < CB; ++b)
        if (c0 + b < nc) {
          const float w = Ws[c0 + b][q];
          o0 += w * x[b].x;
          o1 += w * x[b].y;
        }
    }
    *reinterpret_cast<uint32_t*>(out + (long)(sq.out_row0 + sq.q_begin + q) * ldo + h * HD + d) = pack2(o0, o1);
  }
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
  // the kernel's buffer offsets are 32-bit: a tile's 64 q|k rows, a head's 64 V^T rows
  if (ldqk <= 0 || ld_vt <= 0 || (long)BKV * ldqk * 2 >= (1L << 31) || (long)HD * ld_vt * 2 >= (1L << 31))
    return hipErrorInvalidValue;
  const float scale_log2 = 0.125f * 1.4426950408889634f;  // head_dim^-0.5 * log2(e)
  const long grid = max_items * heads;
  if (grid > 0x7fffffffL) return hipErrorInvalidValue;
  dfh_launch(seq_attention_kernel, dim3((unsigned)grid), dim3(256), 0, s, qk, ldqk, vt, ld_vt, out, ldo, heads,
             reinterpret_cast<const char*>(list), scale_log2, rope_cos, rope_sin);
  return hipGetLastError();
}

hipError_t decode_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                            long ldo, const AttnSeq* seqs, int n_seq, int heads, int max_kv,
                            float* part, unsigned* counters, const float* rope_cos, const float* rope_sin,
                            hipStream_t s) {
  if (n_seq <= 0 || max_kv <= 0) return hipSuccess;
  const float scale_log2 = 0.125f * 1.4426950408889634f;
  const DecodeSplit sp = decode_split(n_seq, heads, max_kv);
  const long groups8 = ((long)n_seq * heads + NXCD - 1) / NXCD * NXCD;
  if (groups8 * sp.n_chunks > 0x7fffffffL) return hipErrorInvalidValue;
  dfh_launch(decode_attention_kernel<kDecodeWaves, kDecodeStages>, dim3((unsigned)(groups8 * sp.n_chunks)),
             dim3(64 * kDecodeWaves), 0, s, qk, ldqk, vt,
             ld_vt, seqs, heads, n_seq * heads, sp.n_chunks, sp.chunk_keys, scale_log2, part, counters, out, ldo,
             rope_cos, rope_sin);
  return hipGetLastError();
}

DecodeSplit decode_split(int n_seq, int heads, int max_kv) {
  // about one workgroup per CU (each holds 128 KB of tiles), chunks of whole
  // rounds of one 64-key tile per wave
  const long groups = (long)n_seq * heads;
  int want = (int)(cu_count() / (groups > 0 ? groups : 1));
  const int rounds = (max_kv + kDecodeWaves * BKV - 1) / (kDecodeWaves * BKV);
  want = std::max(1, std::min(std::min(want, rounds), kDecodeMaxChunks));
  DecodeSplit sp;
  sp.chunk_keys = (rounds + want - 1) / want * (kDecodeWaves * BKV);
  sp.n_chunks = (max_kv + sp.chunk_keys - 1) / sp.chunk_keys;
  return sp;
}

}  // namespace dfh
