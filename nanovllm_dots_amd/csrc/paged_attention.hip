// Paged KV cache of the LLM backbone (Qwen2.5-1.5B: 12 query heads, 2 KV heads,
// head_dim 128, pages of 256 tokens): the cache write and the attention of newly
// appended tokens over the cache.
//
// store_kvcache (nanovllm_dots/layers/attention.py:10-47): token i's K and V
// rows (D = kv_heads * head_dim contiguous bf16) go to cache row slot[i] of
// k_cache / v_cache ([num_slots, D]); slot -1 skips the token. One wave per
// token, 16-B copies.
//
// Paged attention: flash_attn_varlen_func / flash_attn_with_kvcache as
// layers/attention.py:66-95 call them. Sequence i has Lq_i new query tokens
// (rows cu_q[i] .. cu_q[i+1] of q) and Lk_i keys (Lk_i >= Lq_i, the new tokens
// last, already written by store_kvcache). Key t of sequence i lives in
// physical page block_table[i][t / page] at offset t % page, or, without a
// block table, at row cu_k[i] + t of a contiguous K / V. Causal masking is
// bottom-right aligned (flash-attn's convention for Lq < Lk, which is append
// semantics): query token j sees keys [0, Lk - Lq + j]. Query head h uses KV
// head h / G, G = heads / kv_heads.
//
// Work split (split-KV): one workgroup = one wave = 32 query rows (8 when every
// sequence has at most 8: decode with a GQA group <= 8) of one (sequence, KV head) against one chunk of 256 keys (wider past 32 K keys, so
// a row has at most 128 chunks). A row is a (token, head
// within the group) pair, so at decode one wave serves the G heads that share
// the KV head, and K / V are read once for all of them. Inside the chunk the
// wave walks four 64-key tiles with an online softmax: S^T = K Q^T on MFMA
// (32 keys x 32 rows per block, K and Q straight from global memory, 16 B per
// lane), P^T to LDS, then O += P V on the VALU with each lane owning head_dim/64
// columns of O and reading V rows coalesced (the MFMA operand layout would need
// V transposed; at <= 32 rows this product is small next to the K / V bytes).
// In 8-row tiles the next tile's K and V are requested while this tile is computed.
// Each chunk writes (max, sum, O) per row to the workspace; a combine kernel
// merges the chunks of a row and writes bf16. Pages are multiples of 256
// tokens, so a 64-key tile never straddles a page.
#include <type_traits>

#include "dfh_device.h"
#include "dfh_kernels.h"

namespace dfh {

namespace {

constexpr int PCH = 256;  // keys per chunk unit (a chunk is a multiple of it)
constexpr int kMaxChunks = 128;  // chunks per row at most (the chunk widens past 32 K keys)
constexpr int PT = 64;    // keys per tile
constexpr int PR = 32;    // query rows per workgroup

struct PagedParams {
  const uint16_t* q;
  long q_stride;
  const uint16_t* k;
  const uint16_t* v;
  long kv_stride;
  const int* cu_q;
  const int* cu_k;
  const int* seqlens_k;
  const int* block_table;
  int bt_stride, block_size;
  uint16_t* out;
  long out_stride;
  float* ws;
  int kv_heads, group, n_tiles, n_chunks, chunk;  // chunk: keys per workgroup (multiple of PCH)
  float scale_log2;
  int causal;
};

__device__ __forceinline__ int seq_lk(const PagedParams& a, int i) {
  return a.seqlens_k ? a.seqlens_k[i] : a.cu_k[i + 1] - a.cu_k[i];
}

// cache row of key t of sequence i
__device__ __forceinline__ long key_row(const PagedParams& a, int i, int t) {
  if (a.block_table) {
    const int page = a.block_table[(long)i * a.bt_stride + t / a.block_size];
    return (long)page * a.block_size + t % a.block_size;
  }
  return (long)a.cu_k[i] + t;
}

// workspace floats of one (row tile, KV head, chunk) partial of an NR-row tile:
// max[NR], sum[NR], O[NR][HD]
template <int HD, int NR>
constexpr int part_floats() { return 2 * NR + NR * HD; }

// NR query rows per workgroup: 32, or 8 when a sequence's tile has at most 8
// rows (decode with a GQA group <= 8), which keeps O in 16 registers per lane
template <int HD, int NR>
__global__ void __launch_bounds__(64) paged_attention_kernel(PagedParams a) {
  constexpr int KK = HD / 16;  // MFMA k-steps over the head dim
  constexpr int DPL = HD / 64; // O columns per lane
  __shared__ __align__(16) float Ps[PT][NR];  // P^T of the current tile: [key][row]
  __shared__ __align__(16) float As[NR];      // per-row rescale of O for the current tile
  const int lane = threadIdx.x, l32 = lane & 31, hi = lane >> 5;
  const int c = blockIdx.x % a.n_chunks;
  const int it = blockIdx.x / a.n_chunks;  // sequence * n_tiles + row tile
  const int i = it / a.n_tiles, tile = it % a.n_tiles;
  const int g = blockIdx.y;
  const int q0 = a.cu_q[i];
  const int Lq = a.cu_q[i + 1] - q0;
  const int Lk = seq_lk(a, i);
  const int G = a.group;
  const int R = min(NR, Lq * G - tile * NR);  // rows of this tile (uniform)
  if (R <= 0 || c * a.chunk >= Lk) return;
  float* part = a.ws + ((long)(it * a.kv_heads + g) * a.n_chunks + c) * part_floats<HD, NR>();
  // this lane's row (clamped to the last real row) and its visible-key limit
  const int r_me = min(l32, R - 1);
  const int gr = tile * NR + r_me;
  const int j = gr / G, gh = gr % G;
  const int lim = a.causal ? min(Lk, Lk - Lq + j + 1) : Lk;
  // the tile's largest limit: chunks beyond it hold no visible key
  const int j_max = (tile * NR + R - 1) / G;
  const int lim_max = a.causal ? min(Lk, Lk - Lq + j_max + 1) : Lk;
  const int k0 = c * a.chunk;
  if (k0 >= lim_max) {
    if (hi == 0 && l32 < R) {
      part[l32] = -INFINITY;
      part[NR + l32] = 0.f;
    }
    return;
  }
  // Q fragments (B operand): row l32, dims 16*kk + 8*hi .. +8
  bf16x8 qf[KK];
  {
    const uint16_t* qp = a.q + (long)(q0 + j) * a.q_stride + (long)(g * G + gh) * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qp + 16 * kk);
  }
  // In 8-row tiles the K and V of one tile live in registers: the next tile's K
  // is requested right after this tile's S = K Q^T, its V right after this
  // tile's P V, and its page is looked up one tile ahead, so a tile waits on one
  // memory round trip at most. 32-row tiles hold O in 64 registers per lane;
  // there K is loaded per 32-key block just before its MFMAs and V after them,
  // which keeps two waves per SIMD.
  constexpr bool ahead = NR == 8;
  using VT = typename std::conditional<DPL == 2, uint32_t, uint16_t>::type;
  bf16x8 kf[ahead ? 2 : 1][KK];  // block kb: keys kb*32 + l32, dims 16*kk + 8*hi .. +8
  VT vr[PT];                     // key t: this lane's DPL columns
  auto load_kb = [&](int slot, long row0, int last, int kb) {
    const int kt = min(kb * 32 + l32, last);  // keys past Lk read the last key (masked)
    const uint16_t* kp = a.k + (row0 + kt) * a.kv_stride + (long)g * HD + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) kf[slot][kk] = *reinterpret_cast<const bf16x8*>(kp + 16 * kk);
  };
  auto load_v = [&](long row0, int last) {
#pragma unroll
    for (int t = 0; t < PT; ++t)
      vr[t] = *reinterpret_cast<const VT*>(a.v + (row0 + min(t, last)) * a.kv_stride + (long)g * HD + DPL * lane);
  };
  float m_run = -INFINITY, l_run = 0.f;  // row l32's running max / sum (both halves agree)
  float o[NR][DPL];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[r][e] = 0.f;
  const int kend = min(k0 + a.chunk, lim_max);
  if (ahead) {
    const long row0 = key_row(a, i, k0);
    load_kb(0, row0, Lk - 1 - k0, 0);
    load_kb(ahead ? 1 : 0, row0, Lk - 1 - k0, 1);
    load_v(row0, Lk - 1 - k0);
  }
  for (int t0 = k0; t0 < kend; t0 += PT) {
    const int tn = t0 + PT;
    const bool more = ahead && tn < kend;  // uniform
    const long row_n = more ? key_row(a, i, tn) : 0;
    const long row0 = ahead ? 0 : key_row(a, i, t0);
    // S^T = K Q^T: block kb holds keys t0 + kb*32 + [0, 32)
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      if (!ahead) load_kb(0, row0, Lk - 1 - t0, kb);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ahead ? kb : 0][kk], qf[kk], s[kb], 0, 0, 0);
    }
    if (more) {
      load_kb(0, row_n, Lk - 1 - tn, 0);
      load_kb(ahead ? 1 : 0, row_n, Lk - 1 - tn, 1);
    }
    if (!ahead) load_v(row0, Lk - 1 - t0);  // requested before the softmax
    // scores of row l32: lane holds keys kb*32 + 8*(e/4) + 4*hi + e%4
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = t0 + kb * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
        const float sv = key < lim ? s[kb][e] * a.scale_log2 : -INFINITY;
        s[kb][e] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // nothing visible yet in this row
    const float alpha = m_run == -INFINITY ? 0.f : exp2f(m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = exp2f(s[kb][e] - m_use);
        psum += p;
        if (NR == 32 || l32 < NR) Ps[kb * 32 + 8 * (e >> 2) + 4 * hi + (e & 3)][l32] = p;
      }
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (hi == 0 && l32 < NR) As[l32] = alpha;
    __syncthreads();
    // O[r][d] = alpha[r] * O[r][d] + sum_t P[r][t] V[t][d], rows in groups of 8
#pragma unroll
    for (int rb = 0; rb < NR / 8; ++rb) {
      if (rb * 8 >= R) break;  // uniform
      const float4 a0 = *reinterpret_cast<const float4*>(&As[rb * 8]);
      const float4 a1 = *reinterpret_cast<const float4*>(&As[rb * 8 + 4]);
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[rb * 8 + r][e] *= av[r];
#pragma unroll 8
      for (int t = 0; t < PT; ++t) {
        const float4 p0 = *reinterpret_cast<const float4*>(&Ps[t][rb * 8]);
        const float4 p1 = *reinterpret_cast<const float4*>(&Ps[t][rb * 8 + 4]);
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        float vv[DPL];
        if constexpr (DPL == 2) {
          vv[0] = __uint_as_float(vr[t] << 16);
          vv[1] = __uint_as_float(vr[t] & 0xffff0000u);
        } else {
          vv[0] = bf2f(vr[t]);
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
          for (int e = 0; e < DPL; ++e) o[rb * 8 + r][e] = fmaf(pv[r], vv[e], o[rb * 8 + r][e]);
      }
    }
    if (more) load_v(row_n, Lk - 1 - tn);
    __syncthreads();  // Ps / As are rewritten by the next tile
  }
  if (hi == 0 && l32 < R) {
    part[l32] = m_run;
    part[NR + l32] = l_run;
  }
  float* po = part + 2 * NR;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (r >= R) break;  // uniform
    if constexpr (DPL == 2) {
      *reinterpret_cast<float2*>(po + r * HD + 2 * lane) = make_float2(o[r][0], o[r][1]);
    } else {
      po[r * HD + lane] = o[r][0];
    }
  }
}

// Merge the chunks of each row: O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.
// One workgroup per (sequence, row tile, KV head). Every (row, chunk) max and
// sum is loaded once, in parallel, into LDS and turned into a weight there; the
// O reads of a thread do not depend on each other, so they are issued back to
// back. A row that sees no key is 0. At most kMaxChunks chunks per row (the
// launcher widens chunks to keep it so).
template <int HD, int NR>
__global__ void __launch_bounds__(256) paged_combine_kernel(PagedParams a) {
  __shared__ float Ms[NR][kMaxChunks + 1];  // chunk maxima, then weights
  __shared__ float Ls[NR][kMaxChunks + 1];
  const int it = blockIdx.x, g = blockIdx.y;
  const int i = it / a.n_tiles, tile = it % a.n_tiles;
  const int q0 = a.cu_q[i];
  const int Lq = a.cu_q[i + 1] - q0;
  const int Lk = seq_lk(a, i);
  const int G = a.group;
  const int R = min(NR, Lq * G - tile * NR);
  if (R <= 0) return;
  // chunks launched for this row (keys past max_k, a caller error, are not seen)
  const int nc = min((Lk + a.chunk - 1) / a.chunk, a.n_chunks);
  constexpr int PF = part_floats<HD, NR>();
  const float* pp = a.ws + (long)(it * a.kv_heads + g) * a.n_chunks * PF;
  const int tid = threadIdx.x;
  for (int idx = tid; idx < R * nc; idx += 256) {
    const int r = idx % R, cc = idx / R;
    const float* p = pp + (long)cc * PF;
    Ms[r][cc] = p[r];
    Ls[r][cc] = p[NR + r];
  }
  __syncthreads();
  if (tid < R) {
    float M = -INFINITY;
    for (int cc = 0; cc < nc; ++cc) M = fmaxf(M, Ms[tid][cc]);
    float L = 0.f;
    if (M != -INFINITY)
      for (int cc = 0; cc < nc; ++cc)
        if (Ms[tid][cc] != -INFINITY) L += Ls[tid][cc] * exp2f(Ms[tid][cc] - M);
    for (int cc = 0; cc < nc; ++cc)
      Ms[tid][cc] = (L > 0.f && Ms[tid][cc] != -INFINITY) ? exp2f(Ms[tid][cc] - M) / L : 0.f;
  }
  __syncthreads();
  for (int e = tid; e < R * HD; e += 256) {
    const int r = e / HD, d = e % HD;
    const float* po = pp + 2 * NR + r * HD + d;
    float o = 0.f;
#pragma unroll 8
    for (int cc = 0; cc < nc; ++cc) {
      const float w = Ms[r][cc];
      const float x = po[(long)cc * PF];
      o += w != 0.f ? w * x : 0.f;
    }
    const int gr = tile * NR + r;
    const int j = gr / G, gh = gr % G;
    a.out[(long)(q0 + j) * a.out_stride + (long)(g * G + gh) * HD + d] = f2bf(o);
  }
}

__global__ void __launch_bounds__(256)
store_kvcache_kernel(const uint16_t* __restrict__ key, long key_stride, const uint16_t* __restrict__ value,
                     long value_stride, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                     const int* __restrict__ slots, int n, int D) {
  const int lane = threadIdx.x & 63;
  const long idx = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (idx >= n) return;
  const int slot = slots[idx];
  if (slot < 0) return;
  const uint16_t* kp = key + idx * key_stride;
  const uint16_t* vp = value + idx * value_stride;
  uint16_t* kc = k_cache + (long)slot * D;
  uint16_t* vc = v_cache + (long)slot * D;
  for (int col = lane * 8; col < D; col += 64 * 8) {
    *reinterpret_cast<uint4*>(kc + col) = *reinterpret_cast<const uint4*>(kp + col);
    *reinterpret_cast<uint4*>(vc + col) = *reinterpret_cast<const uint4*>(vp + col);
  }
}

}  // namespace

// keys per workgroup for a longest sequence of max_k keys: PCH, widened so a row
// has at most kMaxChunks chunks
int chunk_keys(int max_k) {
  const long units = ((long)max_k + PCH - 1) / PCH;
  return (int)((units + kMaxChunks - 1) / kMaxChunks) * PCH;
}

// sized for 32-row tiles, which also bounds the 8-row tiles of decode
long paged_attention_ws_floats(int batch, int kv_heads, int group, int max_q, int max_k, int head_dim) {
  const long n_tiles = ((long)max_q * group + PR - 1) / PR;
  const long n_chunks = ((long)max_k + chunk_keys(max_k) - 1) / chunk_keys(max_k);
  return (long)batch * n_tiles * kv_heads * n_chunks * (2 * PR + (long)PR * head_dim);
}

hipError_t paged_attention(const PagedAttnArgs& x, hipStream_t s) {
  if (x.head_dim != 64 && x.head_dim != 128) return hipErrorInvalidValue;
  if (x.batch <= 0 || x.kv_heads <= 0 || x.heads % x.kv_heads != 0) return hipErrorInvalidValue;
  if (x.max_q <= 0 || x.max_k <= 0) return hipSuccess;
  PagedParams a{};
  a.q = x.q; a.q_stride = x.q_stride;
  a.k = x.k; a.v = x.v; a.kv_stride = x.kv_stride;
  a.cu_q = x.cu_q; a.cu_k = x.cu_k; a.seqlens_k = x.seqlens_k;
  a.block_table = x.block_table; a.bt_stride = x.bt_stride; a.block_size = x.block_size;
  a.out = x.out; a.out_stride = x.out_stride;
  a.ws = x.ws;
  a.kv_heads = x.kv_heads;
  a.group = x.heads / x.kv_heads;
  // a tile of 8 rows when every sequence's new rows fit one (decode, GQA group <= 8)
  const int nr = (long)x.max_q * a.group <= 8 ? 8 : PR;
  a.n_tiles = (int)(((long)x.max_q * a.group + nr - 1) / nr);
  a.chunk = chunk_keys(x.max_k);
  a.n_chunks = (x.max_k + a.chunk - 1) / a.chunk;
  a.scale_log2 = x.scale * 1.4426950408889634f;
  a.causal = x.causal;
  const long items = (long)x.batch * a.n_tiles;
  if (items * a.n_chunks > 0x7fffffffL || x.kv_heads > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(items * a.n_chunks), (unsigned)x.kv_heads);
  const dim3 cgrid((unsigned)items, (unsigned)x.kv_heads);
  auto run = [&](auto attn, auto combine) {
    dfh_launch(attn, grid, dim3(64), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(combine, cgrid, dim3(256), 0, s, a);
    return hipGetLastError();
  };
  if (x.head_dim == 128)
    return nr == 8 ? run(paged_attention_kernel<128, 8>, paged_combine_kernel<128, 8>)
                   : run(paged_attention_kernel<128, PR>, paged_combine_kernel<128, PR>);
  return nr == 8 ? run(paged_attention_kernel<64, 8>, paged_combine_kernel<64, 8>)
                 : run(paged_attention_kernel<64, PR>, paged_combine_kernel<64, PR>);
}

hipError_t store_kvcache(const uint16_t* key, long key_stride, const uint16_t* value, long value_stride,
                         uint16_t* k_cache, uint16_t* v_cache, const int* slots, int n, int D, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (D % 8 != 0 || key_stride % 8 != 0 || value_stride % 8 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(store_kvcache_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, key, key_stride, value,
                     value_stride, k_cache, v_cache, slots, n, D);
  return hipGetLastError();
}

}  // namespace dfh
