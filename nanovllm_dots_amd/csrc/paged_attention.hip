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
// Work split (split-KV): one workgroup = one wave = 32 query rows of one
// (sequence, KV head) against one chunk of keys. The (sequence, row tile) items
// are a compact list that a one-workgroup plan kernel writes from cu_seqlens_q
// (at most ceil(total_q * G / 32) + batch of them, so a batch of one long and
// many short prompts is not padded to the longest). The chunk count is chosen to
// fill the GPU with about kTargetWaves workgroups: 256-key chunks for a decode
// of a few dozen sequences, one chunk per row tile once the tiles alone fill it
// (then the kernel writes normalised bf16 rows itself and there is no workspace
// of partial sums and no combine launch). A row is a (token, head within the group)
// pair, so at decode one wave serves the G heads that share the KV head, and
// K / V are read once for all of them. Inside the chunk the wave walks four
// 64-key tiles with an online softmax, both products on MFMA:
//   S^T = K Q^T (32 keys x 32 rows per block, K and Q straight from global
//   memory, 16 B per lane);
//   O += P V with P taken from the S registers as the A operand (keys permuted
//   within each 16-key step, the same way for both operands) and V^T staged in
//   LDS: each lane loads its columns of every V row (coalesced row reads) and
//   writes them transposed, 4 keys per 8-B store.
// With several chunks, each writes (max, sum, O) per row to the workspace and a
// combine kernel merges the chunks of a row and writes bf16. Pages are multiples of 256
// tokens, so a 64-key tile never straddles a page.
#include <mutex>
#include <type_traits>

#include "dfh_device.h"
#include "dfh_kernels.h"

// Workspace of the no-allocation entry point (dfh_paged_attention_noalloc): a
// file-scope device array, one copy per GPU at its own address, held until the
// process ends. Host code uses the address hipGetSymbolAddress returns for the
// current device (paged_scratch), never this name.
static __device__ __align__(256) unsigned char scratch[dfh::kPagedScratchBytes];

namespace dfh {

void* paged_scratch(hipError_t* err) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e = hipErrorInvalidDevice;
  if (e != hipSuccess) {
    *err = e;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return nullptr;
    }
    ptrs[dev] = p;
  }
  *err = hipSuccess;
  return ptrs[dev];
}

namespace {

constexpr int PCH = 256;  // keys per chunk unit (a chunk is a multiple of it)
constexpr int kMaxChunks = 128;  // chunks per row at most (the chunk widens past 32 K keys)
constexpr int PT = 64;    // keys per tile
constexpr int PR = 32;    // query rows per workgroup
constexpr int kCombineSplit = 4;  // column slices of head_dim per combine row tile
constexpr long kTargetWaves = 4096;  // attention workgroups (one wave each) that fill the GPU

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
  float* ws;                      // partial sums (n_chunks > 1)
  const int2* items;             // (sequence, row tile) per item; sequence -1: no work
  int kv_heads, group, n_chunks, chunk;  // chunk: keys per workgroup (multiple of PCH)
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

// workspace floats of one (row tile, KV head, chunk) partial: max[PR], sum[PR], O[PR][HD]
template <int HD>
constexpr int part_floats() { return 2 * PR + PR * HD; }

template <int HD>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) paged_attention_kernel(PagedParams a) {
  constexpr int KK = HD / 16;  // MFMA k-steps over the head dim
  constexpr int DPL = HD / 64; // V columns per lane as loaded
  // V^T of the current tile (pitch PT + 4 keys: the 8-B operand reads of a
  // half-wave hit 64 distinct banks) and the per-row rescale of O
  constexpr int VTP = PT + 4;
  __shared__ __align__(16) uint16_t Vt[HD][VTP];
  __shared__ __align__(16) float As[PR];
  const int lane = threadIdx.x, l32 = lane & 31, hi = lane >> 5;
  const int c = blockIdx.x % a.n_chunks;
  const int it = blockIdx.x / a.n_chunks;  // item
  const int2 item = a.items[it];
  if (item.x < 0) return;
  const int i = item.x, tile = item.y;
  const int g = blockIdx.y;
  const int q0 = a.cu_q[i];
  const int Lq = a.cu_q[i + 1] - q0;
  const int Lk = seq_lk(a, i);
  const int G = a.group;
  const int R = min(PR, Lq * G - tile * PR);  // rows of this tile (uniform)
  const bool direct = a.n_chunks == 1;       // no partial sums: normalise and write bf16 here
  if (R <= 0 || (!direct && c * a.chunk >= Lk)) return;
  float* part = direct ? nullptr : a.ws + ((long)(it * a.kv_heads + g) * a.n_chunks + c) * part_floats<HD>();
  // this lane's row (clamped to the last real row) and its visible-key limit
  const int r_me = min(l32, R - 1);
  const int gr = tile * PR + r_me;
  const int j = gr / G, gh = gr % G;
  const int lim = a.causal ? min(Lk, Lk - Lq + j + 1) : Lk;
  // the tile's largest limit: chunks beyond it hold no visible key
  const int j_max = (tile * PR + R - 1) / G;
  const int lim_max = a.causal ? min(Lk, Lk - Lq + j_max + 1) : Lk;
  const int k0 = c * a.chunk;
  if (!direct && k0 >= lim_max) {
    if (hi == 0 && l32 < R) {
      part[l32] = -INFINITY;
      part[PR + l32] = 0.f;
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
  float m_run = -INFINITY, l_run = 0.f;  // row l32's running max / sum (both halves agree)
  // O in MFMA layout: block db = columns db*32 + l32, rows 8*(e/4) + 4*hi + e%4
  floatx16 o[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  const int kend = min(k0 + a.chunk, lim_max);
  for (int t0 = k0; t0 < kend; t0 += PT) {
    const int last = Lk - 1 - t0;  // keys past Lk read the last key (masked)
    const long row0 = key_row(a, i, t0);
    // S^T = K Q^T: block kb holds keys t0 + kb*32 + [0, 32)
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      const int kt = min(kb * 32 + l32, last);
      const uint16_t* kp = a.k + (row0 + kt) * a.kv_stride + (long)g * HD + 8 * hi;
      bf16x8 kf[KK];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kf[kk] = *reinterpret_cast<const bf16x8*>(kp + 16 * kk);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk], qf[kk], s[kb], 0, 0, 0);
    }
    // V rows of the tile (this lane's DPL columns of each key), requested before the softmax
    using VT = typename std::conditional<DPL == 2, uint32_t, uint16_t>::type;
    VT vr[PT];
#pragma unroll
    for (int t = 0; t < PT; ++t)
      vr[t] = *reinterpret_cast<const VT*>(a.v + (row0 + min(t, last)) * a.kv_stride + (long)g * HD + DPL * lane);
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
        s[kb][e] = p;
      }
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (hi == 0) As[l32] = alpha;
    // V^T[d][t] of the tile: this lane's columns DPL*lane + cc, 4 keys per 8-B write
#pragma unroll
    for (int t = 0; t < PT; t += 4)
#pragma unroll
      for (int cc = 0; cc < DPL; ++cc) {
        uint32_t w0, w1;
        if constexpr (DPL == 2) {
          const uint32_t sel = cc ? 0x07060302u : 0x05040100u;  // high / low halves of two keys
          w0 = __builtin_amdgcn_perm(vr[t + 1], vr[t], sel);
          w1 = __builtin_amdgcn_perm(vr[t + 3], vr[t + 2], sel);
        } else {
          w0 = (uint32_t)vr[t] | ((uint32_t)vr[t + 1] << 16);
          w1 = (uint32_t)vr[t + 2] | ((uint32_t)vr[t + 3] << 16);
        }
        *reinterpret_cast<uint2*>(&Vt[DPL * lane + cc][t]) = make_uint2(w0, w1);
      }
    __syncthreads();
    // O = alpha * O + P V on MFMA. k-step q covers the 16 keys that this lane's
    // S entries e = 8*(q%2) .. +8 of block q/2 hold: for half hi, keys
    // 32*(q/2) + 16*(q%2) + 4*hi + {0..3, 8..11}. The V^T operand takes the same keys.
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const float4 al = *reinterpret_cast<const float4*>(&As[8 * g4 + 4 * hi]);
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) {
        o[db][4 * g4 + 0] *= al.x;
        o[db][4 * g4 + 1] *= al.y;
        o[db][4 * g4 + 2] *= al.z;
        o[db][4 * g4 + 3] *= al.w;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int kb = q >> 1, e0 = 8 * (q & 1);
      const uint4 pw = make_uint4(pack2(s[kb][e0], s[kb][e0 + 1]), pack2(s[kb][e0 + 2], s[kb][e0 + 3]),
                                  pack2(s[kb][e0 + 4], s[kb][e0 + 5]), pack2(s[kb][e0 + 6], s[kb][e0 + 7]));
      const bf16x8 pa = __builtin_bit_cast(bf16x8, pw);
      const int kq = 32 * kb + 16 * (q & 1) + 4 * hi;
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) {
        const uint16_t* vp = &Vt[db * 32 + l32][kq];
        const uint2 v0 = *reinterpret_cast<const uint2*>(vp);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vp + 8);
        const bf16x8 vb = __builtin_bit_cast(bf16x8, make_uint4(v0.x, v0.y, v1.x, v1.y));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa, vb, o[db], 0, 0, 0);
      }
    }
    __syncthreads();  // Vt / As are rewritten by the next tile
  }
  if (direct) {
    // O / l of row r = 8*(e/4) + 4*hi + e%4 (a row that sees no key is 0)
    if (hi == 0) As[l32] = l_run > 0.f ? 1.f / l_run : 0.f;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = 8 * (e >> 2) + 4 * hi + (e & 3);
      if (r >= R) continue;
      const float inv = As[r];
      const int grr = tile * PR + r;
      uint16_t* op = a.out + (long)(q0 + grr / G) * a.out_stride + (long)(g * G + grr % G) * HD + l32;
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) op[db * 32] = f2bf(o[db][e] * inv);
    }
    return;
  }
  if (hi == 0 && l32 < R) {
    part[l32] = m_run;
    part[PR + l32] = l_run;
  }
  float* po = part + 2 * PR;
#pragma unroll
  for (int db = 0; db < HD / 32; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = 8 * (e >> 2) + 4 * hi + (e & 3);
      if (r < R) po[r * HD + db * 32 + l32] = o[db][e];
    }
}

// Merge the chunks of each row: O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.
// One workgroup per (sequence, row tile, KV head). Every (row, chunk) max and
// sum is loaded once, in parallel, into LDS and turned into a weight there; the
// O reads of a thread do not depend on each other, so they are issued back to
// back. A row that sees no key is 0. At most kMaxChunks chunks per row (the
// launcher widens chunks to keep it so). blockIdx.z takes one of kCombineSplit
// column slices of head_dim (each slice recomputes the few weights), so a
// decode of a few dozen sequences still fills the GPU.
template <int HD>
__global__ void __launch_bounds__(256) paged_combine_kernel(PagedParams a) {
  __shared__ float Ms[PR][kMaxChunks + 1];  // chunk maxima, then weights
  __shared__ float Ls[PR][kMaxChunks + 1];
  const int it = blockIdx.x, g = blockIdx.y;
  const int2 item = a.items[it];
  if (item.x < 0) return;
  const int i = item.x, tile = item.y;
  const int q0 = a.cu_q[i];
  const int Lq = a.cu_q[i + 1] - q0;
  const int Lk = seq_lk(a, i);
  const int G = a.group;
  const int R = min(PR, Lq * G - tile * PR);
  if (R <= 0) return;
  // chunks launched for this row (keys past max_k, a caller error, are not seen)
  const int nc = min((Lk + a.chunk - 1) / a.chunk, a.n_chunks);
  constexpr int PF = part_floats<HD>();
  const float* pp = a.ws + (long)(it * a.kv_heads + g) * a.n_chunks * PF;
  const int tid = threadIdx.x;
  for (int idx = tid; idx < R * nc; idx += 256) {
    const int r = idx % R, cc = idx / R;
    const float* p = pp + (long)cc * PF;
    Ms[r][cc] = p[r];
    Ls[r][cc] = p[PR + r];
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
  constexpr int CW = HD / kCombineSplit;  // columns of this workgroup
  for (int e = tid; e < R * CW; e += 256) {
    const int r = e / CW, d = blockIdx.z * CW + e % CW;
    const float* po = pp + 2 * PR + r * HD + d;
    float o = 0.f;
#pragma unroll 8
    for (int cc = 0; cc < nc; ++cc) {
      const float w = Ms[r][cc];
      const float x = po[(long)cc * PF];
      o += w != 0.f ? w * x : 0.f;
    }
    const int gr = tile * PR + r;
    const int j = gr / G, gh = gr % G;
    a.out[(long)(q0 + j) * a.out_stride + (long)(g * G + gh) * HD + d] = f2bf(o);
  }
}

// The (sequence, row tile) items of a batch: sequence i has ceil(Lq_i * G / 32)
// row tiles; items past the batch's total (the list is sized by a host bound)
// are marked with sequence -1. One workgroup; a running offset carries the scan
// of per-sequence tile counts from one block of 256 sequences to the next.
__global__ void __launch_bounds__(256) paged_plan_kernel(const int* __restrict__ cu_q, int batch, int group,
                                                          int n_items, int2* __restrict__ items) {
  __shared__ int scan[256];
  __shared__ int carry;
  const int tid = threadIdx.x;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < batch; b0 += 256) {
    const int i = b0 + tid;
    const int cnt = i < batch ? (int)(((long)(cu_q[i + 1] - cu_q[i]) * group + PR - 1) / PR) : 0;
    scan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // inclusive scan
      const int v = tid >= off ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += v;
      __syncthreads();
    }
    const int start = carry + scan[tid] - cnt;
    for (int t = 0; t < cnt && start + t < n_items; ++t) items[start + t] = make_int2(i, t);
    __syncthreads();
    if (tid == 255) carry += scan[255];
    __syncthreads();
  }
  for (int k = carry + tid; k < n_items; k += 256) items[k] = make_int2(-1, 0);
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

// The work split of one call: items (row tiles) bounded by the padded count
// batch * ceil(max_q * G / 32) and, when the host knows the number of query
// rows, by ceil(total_q * G / 32) + batch; chunks of keys so that items x KV
// heads x chunks is about kTargetWaves (at most ceil(max_k / 256) chunks, and a
// row has at most kMaxChunks of them: wider chunks past 32 K keys).
struct PagedPlan {
  long n_items;
  int n_chunks, chunk;
};
PagedPlan paged_plan(int batch, int kv_heads, int group, int max_q, int max_k, long total_q) {
  PagedPlan p;
  p.n_items = (long)batch * (((long)max_q * group + PR - 1) / PR);
  if (total_q > 0) {
    const long bound = (total_q * group + PR - 1) / PR + batch;
    if (bound < p.n_items) p.n_items = bound;
  }
  const long units = ((long)max_k + PCH - 1) / PCH;
  long nc = (kTargetWaves + p.n_items * kv_heads - 1) / (p.n_items * kv_heads);
  if (nc > units) nc = units;
  if (nc < 1) nc = 1;
  long per = (units + nc - 1) / nc;                                  // 256-key units per chunk
  const long min_per = (units + kMaxChunks - 1) / kMaxChunks;        // at most kMaxChunks chunks
  if (per < min_per) per = min_per;
  p.chunk = (int)(per * PCH);
  p.n_chunks = (int)((max_k + p.chunk - 1) / p.chunk);
  return p;
}

// workspace bytes: the item list (16-B aligned), then the partial sums when a row has several chunks
long paged_attention_ws_bytes(int batch, int kv_heads, int group, int max_q, int max_k, int head_dim, long total_q) {
  const PagedPlan p = paged_plan(batch, kv_heads, group, max_q, max_k, total_q);
  const long list = (p.n_items * 8 + 255) / 256 * 256;
  const long parts = p.n_chunks > 1 ? p.n_items * kv_heads * p.n_chunks * (2 * PR + (long)PR * head_dim) * 4 : 0;
  return list + parts;
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
  a.kv_heads = x.kv_heads;
  a.group = x.heads / x.kv_heads;
  const PagedPlan p = paged_plan(x.batch, x.kv_heads, a.group, x.max_q, x.max_k, x.total_q);
  a.chunk = p.chunk;
  a.n_chunks = p.n_chunks;
  const long list = (p.n_items * 8 + 255) / 256 * 256;
  a.items = reinterpret_cast<const int2*>(x.ws);
  a.ws = reinterpret_cast<float*>(reinterpret_cast<char*>(x.ws) + list);
  a.scale_log2 = x.scale * 1.4426950408889634f;
  a.causal = x.causal;
  if (p.n_items * a.n_chunks > 0x7fffffffL || x.kv_heads > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(paged_plan_kernel, dim3(1), dim3(256), 0, s, x.cu_q, x.batch, a.group, (int)p.n_items,
                     reinterpret_cast<int2*>(x.ws));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)(p.n_items * a.n_chunks), (unsigned)x.kv_heads);
  const dim3 cgrid((unsigned)p.n_items, (unsigned)x.kv_heads, kCombineSplit);
  auto run = [&](auto attn, auto combine) {
    dfh_launch(attn, grid, dim3(64), 0, s, a);
    hipError_t e2 = hipGetLastError();
    if (e2 != hipSuccess || a.n_chunks == 1) return e2;
    hipLaunchKernelGGL(combine, cgrid, dim3(256), 0, s, a);
    return hipGetLastError();
  };
  return x.head_dim == 128 ? run(paged_attention_kernel<128>, paged_combine_kernel<128>)
                           : run(paged_attention_kernel<64>, paged_combine_kernel<64>);
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
