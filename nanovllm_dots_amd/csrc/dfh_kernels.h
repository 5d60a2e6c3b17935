// Host-side launch interface of the FM/DiT head kernels (internal to the library).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dfh {

// Dispatch-packet timing: when both events are set, the next kernel launched by a
// dfh launcher records them (hipExtLaunchKernelGGL) and the slot is cleared.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchEvents g_launch_events;

// launch helper honouring g_launch_events
template <typename K, typename... Args>
inline void dfh_launch(K kernel, dim3 grid, dim3 block, unsigned shmem, hipStream_t s, Args... args);

enum Epilogue : int {
  EPI_BIAS = 0,      // C = bf16(acc + bias)
  EPI_GELU = 1,      // C = bf16(gelu_tanh(bf16(acc + bias)))
  EPI_GATE_RES = 2,  // C = bf16(C + bf16(gate[req(m)] * bf16(acc + bias)))   (in place)
  EPI_QKV = 3,       // q|k -> C (optional qk-norm, RoPE), v -> V^T (transposed)
  EPI_F32 = 4,       // Cf = acc + bias (float32 out; tests)
  EPI_I32 = 5,       // int8 operands: Ci = int32 accumulators
  EPI_DQ = 6,        // int8 operands: C = bf16(((float(acc) * sx[m]) * sw[n]) + bias[n])
  EPI_SILU = 7,      // C = bf16(silu(bf16(acc + bias)))
  // int8 operands, the linear's output dequantised first, y = ((float(acc) * sx[m]) * sw[n]) + bias[n]
  // (int8_dit.py:60-63), then the bf16 epilogue of the same name on bf16(y)
  EPI_DQ_GELU = 8,
  EPI_DQ_GATE_RES = 9,
  EPI_DQ_QKV = 10,
};
// the dequantising epilogues and the bf16 epilogue each continues with
constexpr bool is_dq(int e) { return e == EPI_DQ || e == EPI_DQ_GELU || e == EPI_DQ_GATE_RES || e == EPI_DQ_QKV; }
constexpr int base_epi(int e) {
  return e == EPI_DQ ? EPI_BIAS : e == EPI_DQ_GELU ? EPI_GELU : e == EPI_DQ_GATE_RES ? EPI_GATE_RES
       : e == EPI_DQ_QKV ? EPI_QKV : e;
}

struct GemmArgs {
  const uint16_t* A; long lda;       // [M, K] bf16 activations, K contiguous
  const uint16_t* B; long ldb;       // [N, K] bf16 weights (nn.Linear layout)
  uint16_t* C; long ldc;             // [M, N] bf16 output
  float* Cf;                         // float32 output (EPI_F32)
  int* Ci;                           // int32 output (EPI_I32)
  const float* sx; const float* sw;  // EPI_DQ: per-row and per-column scales
  const uint16_t* bias;              // [N] or null
  int M; const int* M_dev;           // rows; M_dev (device int) overrides M when non-null
  int N, K;
  // EPI_GATE_RES (res: residual source rows, ld_res; null: C itself, updated in place)
  const uint16_t* gate; long ld_gate; const int* row_req;
  const uint16_t* res; long ld_res;
  // EPI_QKV
  int hidden, head_dim;
  const float* rope_cos; const float* rope_sin;  // rope_table layout (grouped by 32 positions) or null
  int rope_q_in_attn;                            // q leaves without RoPE: the attention kernel rotates it
  const int* row_pos;                            // [M] position of each row within its request
  int qk_norm;                                   // 0 none, 1 LayerNorm(affine), 2 RMSNorm
  const uint16_t* qn_w; const uint16_t* qn_b;    // [head_dim]
  const uint16_t* kn_w; const uint16_t* kn_b;
  uint16_t* vt; long ld_vt; const int* vt_col;   // V^T [hidden, ld_vt]; column of row m = vt_col[m]
  const int* c_rows;                             // optional: q|k output row of row m
  int col0;                                      // fused q|k|v column of B's first row (0, or hidden: k|v only)
  // Optional K-split of the last, partial round of tiles: each XCD's leftover
  // tiles are cut along K over its idle workgroups; partial sums go to ws and the
  // workgroup that completes a tile adds them and runs the epilogue. ws_elems
  // (32-bit words) must cover 4096 + grid * BM * BN or the split is off; the
  // first 4096 words are tile counters that must be zero before the first use
  // (they are left at zero).
  float* ws; long ws_elems;
};

// Picks a tile shape for (M, N, K) and launches the persistent MFMA kernel.
// Returns hipSuccess or an error (shape not supported / launch failure).
hipError_t gemm_bf16(const GemmArgs& a, int epi, hipStream_t s, int tile_hint = -1);

// int8 x int8 -> int32 GEMM (A [M, K] int8, B [N, K] int8, K-contiguous) with the
// EPI_I32 or EPI_DQ epilogue. lda/ldb/K are given in BYTES (int8 elements).
hipError_t gemm_i8(const GemmArgs& a, int epi, hipStream_t s, int tile_hint = -1);

// Per-row dynamic int8 quantisation of a bf16 [M, K] matrix (Int8DynamicLinear,
// int8_dit.py:57-58): s = max(bf16(amax/127), bf16(1e-8)); q = clamp(rint(bf16(x/s)), +-127).
hipError_t quant_rows_bf16(const uint16_t* x, long ldx, int8_t* q, long ldq, float* scale, int M, int K,
                           hipStream_t s, const int* M_dev = nullptr);  // M_dev: device row count (M: bound)
// Per-output-channel int8 weight quantisation in float32 (int8_dit.py:40-45).
hipError_t quant_weight_f32(const uint16_t* w, int8_t* q, float* scale, int N, int K, hipStream_t s);

// Row kernels -------------------------------------------------------------------
// LayerNorm (no affine, fp32 stats) + adaLN modulate:
//   out[m] = bf16( LN(x[m]) * bf16(1 + scale[req]) + shift[req] )
// q (with sx, ldq >= H): the bf16 rows also leave per-token quantised, as
// quant_rows_bf16 would quantise them (bit-identical); out may then be null.
hipError_t ln_modulate(const uint16_t* x, long ldx, uint16_t* out, long ldo,
                       const uint16_t* shift, const uint16_t* scale, long ld_mod,
                       const int* row_req, const int* row_map, int rows_upper, const int* M_dev,
                       int H, float eps, hipStream_t s, int8_t* q = nullptr, long ldq = 0,
                       float* sx = nullptr);

// One attention sequence (device array element). Rows index the q|k buffer
// ([rows, ldqk], ldqk >= 2H: q in columns [0, H), k in [H, 2H)); V^T is [H, ld_vt].
struct AttnSeq {
  int q_row0;      // q|k row of query position 0
  int kv_row0;     // q|k row of key position 0
  int vt_col0;     // V^T column of key position 0 (multiple of 8)
  int q_begin, q_end;  // query positions computed
  int causal_end;  // queries below it see keys [0, q]; the others [0, kv_len)
  int kv_len;
  int out_row0;    // output row of query position 0
};

// Work list of seq_attention: word 0 the item count, then from byte 64 one
// AttnItem per 128-query tile of a sequence: sequences by tile count, most
// first, each sequence's tiles together from the highest index (the longest)
// down. At most one item per query row, so
// 64 + 64 * (query rows of all sequences) bytes suffice.
struct AttnItem {
  AttnSeq seq;
  int tile;  // 128-query tile index within the sequence
  int pad[7];
};
constexpr int kAttnListHeader = 64;  // bytes before the first item
hipError_t attention_worklist(const AttnSeq* seqs, int n_seq, void* list, hipStream_t s);

// Varlen attention with the implicit FM mask (head_dim 64), one workgroup per
// 128 queries of one (sequence, head): workgroup v takes item v / heads of
// `list` (attention_worklist of the same sequences), head v % heads.
// max_items bounds the item count of the list (e.g. n_seq * ceil(max_q / 128)).
// rope_cos / rope_sin (rope_table layout, or null): the q rows hold no RoPE yet and
// query position q of a sequence is rotated here, as the QKV epilogue would.
hipError_t seq_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                         long ldo, int heads, const void* list, long max_items, const float* rope_cos,
                         const float* rope_sin, hipStream_t s);

// Split-KV decode attention: every query of a sequence sees all kv_len keys
// (q_begin..q_end are at most 32 queries). Each (sequence, head) is cut into
// decode_split(...).n_chunks chunks of keys read straight from HBM, one
// workgroup each; the last chunk of a (sequence, head) to finish merges the
// chunk partials in `part` and writes the rows. part holds
// n_seq * heads * n_chunks * 32 * 66 floats (n_chunks <= ceil(max_kv / 256));
// counters holds n_seq * heads zeroed words and is left zeroed by every launch.
// Keys are read in whole 64-key tiles: the q|k rows and V^T columns of a
// sequence up to kv_len rounded up to 64 must be readable and finite.
struct DecodeSplit {
  int n_chunks = 1, chunk_keys = 256;
};
DecodeSplit decode_split(int n_seq, int heads, int max_kv);
hipError_t decode_attention(const uint16_t* qk, long ldqk, const uint16_t* vt, long ld_vt, uint16_t* out,
                            long ldo, const AttnSeq* seqs, int n_seq, int heads, int max_kv,
                            float* part, unsigned* counters, const float* rope_cos, const float* rope_sin,
                            hipStream_t s);

// compute units of the current device (queried once)
int cu_count();

// Paged attention of appended tokens over a paged (or contiguous) KV cache
// (flash_attn_varlen_func / flash_attn_with_kvcache semantics, bottom-right
// causal, GQA). head_dim 64 or 128; block_size a multiple of 256 when paged.
struct PagedAttnArgs {
  int batch, heads, kv_heads, head_dim, max_q, max_k;
  long total_q;                  // query rows of the batch (0: unknown, bounded by batch * max_q)
  const uint16_t* q;
  long q_stride;                 // elements between query tokens
  const int* cu_q;               // [batch + 1]
  const uint16_t* k;
  const uint16_t* v;
  long kv_stride;                // elements between key tokens
  const int* cu_k;               // [batch + 1] or null (then seqlens_k)
  const int* seqlens_k;          // [batch] or null
  const int* block_table;        // [batch, bt_stride] or null (contiguous K / V at rows cu_k[i] + t)
  int bt_stride, block_size;
  uint16_t* out;
  long out_stride;
  float scale;
  int causal;
  void* ws;                      // paged_attention_ws_bytes(...) bytes, 256-B aligned
};
long paged_attention_ws_bytes(int batch, int kv_heads, int group, int max_q, int max_k, int head_dim, long total_q);
hipError_t paged_attention(const PagedAttnArgs& a, hipStream_t s);
// the no-allocation entry point's workspace: a static device array of this size,
// its address on the current device (looked up once per device)
constexpr long kPagedScratchBytes = 64L << 20;
void* paged_scratch(hipError_t* err);
// key / value [n, D] rows (strides in elements) -> cache rows slots[i] ([num_slots, D]); slot < 0 skips
hipError_t store_kvcache(const uint16_t* key, long key_stride, const uint16_t* value, long value_stride,
                         uint16_t* k_cache, uint16_t* v_cache, const int* slots, int n, int D, hipStream_t s);

}  // namespace dfh

#include <hip/hip_ext.h>
namespace dfh {
template <typename K, typename... Args>
inline void dfh_launch_with(LaunchEvents& ev, K kernel, dim3 grid, dim3 block, unsigned shmem, hipStream_t s,
                            Args... args) {
  if (ev.start) {
    hipEvent_t a = ev.start, b = ev.stop;
    ev.start = ev.stop = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, a, b, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
  }
}
template <typename K, typename... Args>
inline void dfh_launch(K kernel, dim3 grid, dim3 block, unsigned shmem, hipStream_t s, Args... args) {
  dfh_launch_with(g_launch_events, kernel, grid, block, shmem, s, args...);
}

}  // namespace dfh
