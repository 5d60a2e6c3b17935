// C ABI of the FM/DiT head: handle, weight packing, workspace and the
// graph-free MeanFlow launch sequence.
//
// The solve (batched_meanflow, nanovllm_dots/models/dots/batched_fm.py:82-126, with
// DiT.forward, native/dit.py:135-148, as the velocity predictor) is one straight
// stream-ordered sequence of kernels. Shapes that depend on the request lengths
// (packed row count M, per-request offsets) are computed on the device from
// pos_ids; grids are sized from host-known upper bounds (N*T rows) and every
// kernel reads the device row count, so a new batch shape needs no capture, no
// host sync and no allocation (once the workspace has grown to it).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/dots_fm.h"
#include "dfh_kernels.h"
#include "dfh_ops.h"

namespace dfh {
thread_local LaunchEvents g_launch_events;
}

using namespace dfh;

namespace {

thread_local std::string g_err;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return 1;
}

#define DFH_CHECK(expr)                                                                   \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) return fail("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                      __FILE__, __LINE__);                                \
  } while (0)

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
};

hipError_t dev_alloc(DevBuf& b, size_t bytes) {
  if (b.bytes >= bytes && b.p) return hipSuccess;
  if (b.p) {
    hipError_t e = hipFree(b.p);
    if (e != hipSuccess) return e;
  }
  b.p = nullptr;
  b.bytes = 0;
  if (bytes == 0) return hipSuccess;
  hipError_t e = hipMalloc(&b.p, bytes);
  if (e != hipSuccess) return e;
  b.bytes = bytes;
  return hipMemset(b.p, 0, bytes);
}

template <typename T>
T* P(DevBuf& b) { return reinterpret_cast<T*>(b.p); }

enum ProfClass { PC_QKV = 0, PC_O, PC_FC1, PC_FC2, PC_ATTN, PC_LN, PC_OTHER, PC_TAIL, PC_QUANT, PC_N };

// an int8 linear: weight [N, K] row-major and its per-output-channel scales
struct Q8 {
  const int8_t* w = nullptr;
  const float* s = nullptr;
};

}  // namespace

struct DfhHandle {
  DfhConfig cfg;
  std::vector<float> rope_inv_freq, temb_freqs;
  int ld_mod = 0;  // n_blocks*6H + 2H
  bool weights_set = false;

  // packed weights (bf16)
  DevBuf w_arena;
  const uint16_t *in_w, *in_b, *t_w0, *t_b0, *t_w2, *t_b2, *d_w0, *d_b0, *d_w2, *d_b2;
  const uint16_t *ada_w, *ada_b, *fin_w, *fin_b, *coord_w, *coord_b;
  std::vector<const uint16_t*> qkv_w, qkv_b, o_w, o_b, fc1_w, fc1_b, fc2_w, fc2_b;
  std::vector<const uint16_t*> qn_w, qn_b, kn_w, kn_b;
  DevBuf consts;  // rope inv_freq, temb freqs (float32)

  // workspace capacity
  int cap_n = 0, cap_T = 0, cap_S = 0;
  long cap_M = 0, ld_vt = 0;
  DevBuf seq, x, hbuf, qk, attn, ff, vt;
  DevBuf x0;  // solve: input_layer of every packed row, once per solve (latent rows per step)
  DevBuf row_req, row_pos, vt_col, cu_rows, cu_vt, hist_len, counts, err, patch_rows, seqs;
  DevBuf tail_seqs, tail_req, tail_pos;  // last block on the latent rows: queries, row -> request / position
  DevBuf rope_cos, rope_sin;
  DevBuf temb_in, t_hid, t_out, d_hid, d_out, cond, cond_act, mod;
  DevBuf z, zp, fin, vel, tvals;
  DevBuf splitws;  // K-split: tile counters, then a 256x256 f32 partial tile per resident workgroup
  DevBuf attq;     // attention work list: item count, then one AttnItem per 128-query tile
  bool ksplit = true;
  bool ln_quant = true;  // int8 mode: LayerNorm+modulate also quantises the next linear's input rows
  bool latent_tail = true;  // solve: the last block's attention / O / MLP on the latent rows only

  // W8A8 mode (Int8DynamicLinear / quantize_dit_, int8_dit.py:34-85): every DiT
  // linear with min(in, out) >= 512 has an int8 weight with per-output-channel
  // scales; the input rows of each are quantised per token right before its GEMM
  // (the q, k and v projections share their input and with it its quantisation)
  bool int8 = false;
  DevBuf w8;                          // the int8 weights and scales
  Q8 in_q, t2_q, d2_q, ada_q;         // input_layer, time / duration MLP second linears, stacked adaLN
  std::vector<Q8> qkv_q, o_q, fc1_q, fc2_q;
  DevBuf aq, asx;                     // quantised input rows of the current GEMM and their scales
  long aq_rows = 0;

  // profiling
  bool prof = false;
  unsigned prof_mask = ~0u;  // classes whose launches carry events
  int prof_every = 1;        // of those, every prof_every-th launch of its class
  long prof_seen[PC_N] = {0};
  std::vector<hipEvent_t> ev_pool;
  std::vector<std::pair<int, int>> ev_used;  // (class, pool index of start)
  size_t ev_next = 0;
  double prof_ms[PC_N] = {0};
  long prof_n[PC_N] = {0};
};

namespace {

// arm dispatch-packet events for the next launch of class `pc`
void prof_arm(DfhHandle* h, int pc) {
  if (!h->prof || !((h->prof_mask >> pc) & 1u)) return;
  if (h->prof_seen[pc]++ % h->prof_every) return;
  if (h->ev_next + 2 > h->ev_pool.size()) return;  // pool full: drop the sample
  const int i = (int)h->ev_next;
  h->ev_next += 2;
  g_launch_events.start = h->ev_pool[i];
  g_launch_events.stop = h->ev_pool[i + 1];
  h->ev_used.push_back({pc, i});
}

int check_cfg(const DfhConfig& c) {
  if (c.head_dim != 64) return fail("head_dim must be 64 (got %d)", c.head_dim);
  if (c.heads * c.head_dim != c.hidden) return fail("heads*head_dim != hidden");
  if (c.hidden % 256 || c.ffn % 256) return fail("hidden and ffn must be multiples of 256");
  if (c.hidden > 2048) return fail("hidden > 2048 not supported");
  if (c.latent_dim % 64) return fail("latent_dim must be a multiple of 64");
  if (c.freq_dim % 64 || c.freq_dim <= 0) return fail("freq_dim must be a positive multiple of 64");
  if (c.n_blocks <= 0 || c.patch <= 0) return fail("n_blocks and patch must be positive");
  if (c.qk_norm < 0 || c.qk_norm > 2) return fail("qk_norm must be 0, 1 or 2");
  if (c.rotary && !c.rope_inv_freq) return fail("rotary requires rope_inv_freq");
  if (!c.temb_freqs) return fail("temb_freqs is required");
  return 0;
}

hipError_t gemm(DfhHandle* h, int pc, const GemmArgs& a_in, int epi, hipStream_t s, int tile = -1) {
  prof_arm(h, pc);
  GemmArgs a = a_in;
  if (h->ksplit) {
    a.ws = P<float>(h->splitws);  // K-split of the last partial round of tiles
    a.ws_elems = (long)(h->splitws.bytes / 4);
  }
  return gemm_bf16(a, epi, s, tile);
}

// int8 mode: room for the quantised input rows of any GEMM on `rows` rows (K <= max(hidden, ffn))
int reserve_q8(DfhHandle* h, long rows, hipStream_t s) {
  if (!h->int8 || rows <= h->aq_rows) return 0;
  DFH_CHECK(hipStreamSynchronize(s));
  const long K = h->cfg.ffn > h->cfg.hidden ? h->cfg.ffn : h->cfg.hidden;
  DFH_CHECK(dev_alloc(h->aq, rows * K));
  DFH_CHECK(dev_alloc(h->asx, rows * 4));
  h->aq_rows = rows;
  return 0;
}

// A linear layer: the bf16 GEMM, or in int8 mode with an int8 weight q, the
// input rows quantised per token (bit-exact with int8_dit.py:57-58) and the i8
// GEMM with the epilogue that dequantises first ((acc * s_x) * s_w) + b.
// a_ready: the input rows are already quantised in h->aq / h->asx (by the
// LayerNorm+modulate that produced them, ln_q8); a.A is then not read.
hipError_t lin(DfhHandle* h, int pc, const GemmArgs& a, int epi, const Q8& q, hipStream_t s, int tile = -1,
               bool a_ready = false) {
  if (!h->int8 || !q.w) return gemm(h, pc, a, epi, s, tile);
  if (a.M > h->aq_rows || (long)a.K > (h->cfg.ffn > h->cfg.hidden ? h->cfg.ffn : h->cfg.hidden))
    return hipErrorInvalidValue;  // reserve_q8 sizes the rows beforehand
  int8_t* aq = P<int8_t>(h->aq);
  float* sx = P<float>(h->asx);
  if (!a_ready) {
    prof_arm(h, PC_QUANT);
    hipError_t e = quant_rows_bf16(a.A, a.lda, aq, a.K, sx, a.M, a.K, s, a.M_dev);
    if (e != hipSuccess) return e;
  }
  GemmArgs b = a;
  b.A = reinterpret_cast<const uint16_t*>(aq); b.lda = a.K;   // bytes
  b.B = reinterpret_cast<const uint16_t*>(q.w); b.ldb = a.K;
  b.sx = sx; b.sw = q.s;
  const int epi8 = epi == EPI_BIAS ? EPI_DQ : epi == EPI_GELU ? EPI_DQ_GELU : epi == EPI_GATE_RES ? EPI_DQ_GATE_RES
                 : epi == EPI_QKV ? EPI_DQ_QKV : -1;
  if (epi8 < 0) return hipErrorInvalidValue;
  prof_arm(h, pc);
  if (h->ksplit) {
    b.ws = P<float>(h->splitws);
    b.ws_elems = (long)(h->splitws.bytes / 4);
  }
  return gemm_i8(b, epi8, s, tile);
}

// LayerNorm + modulate of the rows that feed the linear with int8 weight q. In
// int8 mode (and with the fused quantiser on) the rows also leave quantised in
// h->aq / h->asx for lin(..., a_ready = true); keep_bf16 = false skips the bf16
// rows when nothing else reads them. Returns whether the rows are quantised.
bool ln_q8(DfhHandle* h, const uint16_t* x, uint16_t* out, const uint16_t* shift, const uint16_t* scale,
           long ldm, const int* row_req, int Mup, const int* Md, const Q8& q, bool keep_bf16, hipStream_t s,
           hipError_t* err) {
  const DfhConfig& c = h->cfg;
  const int H = c.hidden;
  const bool fuse = h->int8 && q.w && h->ln_quant && Mup <= h->aq_rows;
  prof_arm(h, PC_LN);
  *err = ln_modulate(x, H, (fuse && !keep_bf16) ? nullptr : out, H, shift, scale, ldm, row_req, nullptr, Mup, Md,
                     H, c.ln_eps, s, fuse ? P<int8_t>(h->aq) : nullptr, H, fuse ? P<float>(h->asx) : nullptr);
  return fuse;
}

// Tile shape per GEMM role (indices of gemm_bf16's configurations), chosen from
// measured throughput at M ~ 37k rows: 8-wave 256x256 tiles whose K-step DMA is
// issued by one half of the workgroup for the fused QKV, the wide (N=4096) and the
// deep (K=4096) products; two 128x128 workgroups per CU for N=1024, K=1024 (their
// epilogues overlap the other workgroup's MFMAs; 256-wide tiles would leave a third
// of the last round idle).
enum GemmRole { kRoleQKV, kRoleNarrow, kRoleWide };
int tile_for(long M, int N, int K, GemmRole role) {
  if (M < 4096) return -1;  // small problems: the library heuristic
  if (role == kRoleQKV) return N % 256 == 0 ? 8 : 2;
  if (role == kRoleWide) return N % 256 == 0 ? 8 : -1;
  if (K >= 4096 && N % 256 == 0) return 8;
  // narrow outputs (N = hidden) at K = hidden: 128x128 tiles, two workgroups per
  // CU; 256-wide tiles (N/256 column blocks) leave up to a third of the last round idle
  return (N % 128 == 0 && K % 64 == 0) ? 2 : -1;
}

GemmArgs linear_args(const uint16_t* A, long lda, const uint16_t* W, const uint16_t* b, uint16_t* C,
                     long ldc, int M, const int* M_dev, int N, int K) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = A; a.lda = lda; a.B = W; a.ldb = K; a.C = C; a.ldc = ldc; a.bias = b;
  a.M = M; a.M_dev = M_dev; a.N = N; a.K = K;
  return a;
}

// Row stride of the q|k buffers (elements): 2H plus 64. With a stride of
// exactly 2H (4 KB at H = 1024), a head's 128-B key slices in consecutive rows
// fall in the same few HBM channels; the padding walks them across the
// channels (decode attention at 4 x 10,111 cached keys: 39.5 -> 35.8 us per
// layer on one box).
long qk_stride(const DfhConfig& c) { return 2L * c.hidden + 64; }

// row-sized workspace (packed rows of one pass)
int reserve_rows(DfhHandle* h, long M, hipStream_t s) {
  if (M <= h->cap_M) return 0;
  const DfhConfig& c = h->cfg;
  DFH_CHECK(hipStreamSynchronize(s));  // in-flight kernels may still use the old buffers
  const long H = c.hidden, F = c.ffn, ld = c.latent_dim;
  DFH_CHECK(dev_alloc(h->seq, M * H * 2));
  DFH_CHECK(dev_alloc(h->x, M * H * 2));
  DFH_CHECK(dev_alloc(h->x0, M * H * 2));
  DFH_CHECK(dev_alloc(h->hbuf, M * H * 2));
  DFH_CHECK(dev_alloc(h->qk, M * qk_stride(c) * 2));
  DFH_CHECK(dev_alloc(h->attn, M * H * 2));
  DFH_CHECK(dev_alloc(h->ff, M * F * 2));
  DFH_CHECK(dev_alloc(h->row_req, M * 4));
  DFH_CHECK(dev_alloc(h->row_pos, M * 4));
  DFH_CHECK(dev_alloc(h->attq, kAttnListHeader + M * sizeof(AttnItem)));  // at most one item per query row
  DFH_CHECK(dev_alloc(h->vt_col, M * 4));
  DFH_CHECK(dev_alloc(h->fin, M * H * 2));
  DFH_CHECK(dev_alloc(h->vel, M * ld * 2));
  if (!h->splitws.p) {
    int dev = 0, cus = 0;
    DFH_CHECK(hipGetDevice(&dev));
    DFH_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // 4096 tile counters, then one 256x256 f32 partial tile per resident workgroup (zeroed)
    DFH_CHECK(dev_alloc(h->splitws, ((size_t)4096 + (size_t)cus * 256 * 256) * 4));
  }
  h->cap_M = M;
  return reserve_q8(h, M, s);
}

int reserve(DfhHandle* h, int n, int T, int S, hipStream_t s) {
  const DfhConfig& c = h->cfg;
  if (reserve_rows(h, (long)n * T, s)) return 1;
  if (n <= h->cap_n && T <= h->cap_T && S <= h->cap_S && h->ld_vt >= (long)n * T + 8L * n + 128) return 0;
  DFH_CHECK(hipStreamSynchronize(s));
  const int nn = n > h->cap_n ? n : h->cap_n;
  const int TT = T > h->cap_T ? T : h->cap_T;
  const int SS = S > h->cap_S ? S : h->cap_S;
  const long M = (long)nn * TT;
  const long H = c.hidden, P = c.patch, ld = c.latent_dim;
  const long ld_vt = M + 8L * nn + 128;
  DFH_CHECK(dev_alloc(h->vt, (size_t)H * ld_vt * 2));
  DFH_CHECK(dev_alloc(h->cu_rows, (nn + 1) * 4));
  DFH_CHECK(dev_alloc(h->cu_vt, (nn + 1) * 4));
  DFH_CHECK(dev_alloc(h->hist_len, nn * 4));
  DFH_CHECK(dev_alloc(h->counts, 16));
  DFH_CHECK(dev_alloc(h->err, 16));
  DFH_CHECK(dev_alloc(h->patch_rows, nn * P * 4));
  DFH_CHECK(dev_alloc(h->seqs, (long)nn * SS * sizeof(AttnSeq)));
  DFH_CHECK(dev_alloc(h->tail_seqs, (long)nn * sizeof(AttnSeq)));
  DFH_CHECK(dev_alloc(h->tail_req, (long)nn * P * 4));
  DFH_CHECK(dev_alloc(h->tail_pos, (long)nn * P * 4));
  DFH_CHECK(dev_alloc(h->rope_cos, (size_t)((TT + 31) / 32) * 32 * 32 * 4));  // whole 32-position groups
  DFH_CHECK(dev_alloc(h->rope_sin, (size_t)((TT + 31) / 32) * 32 * 32 * 4));
  const long RS = (long)SS > nn ? SS : nn;  // timestep rows: per step (solve) or per request (forward)
  DFH_CHECK(dev_alloc(h->temb_in, RS * c.freq_dim * 2));
  DFH_CHECK(dev_alloc(h->t_hid, RS * H * 2));
  DFH_CHECK(dev_alloc(h->t_out, RS * H * 2));
  DFH_CHECK(dev_alloc(h->d_hid, RS * H * 2));
  DFH_CHECK(dev_alloc(h->d_out, RS * H * 2));
  DFH_CHECK(dev_alloc(h->cond, (long)SS * nn * H * 2));
  DFH_CHECK(dev_alloc(h->cond_act, (long)SS * nn * H * 2));
  DFH_CHECK(dev_alloc(h->mod, (long)SS * nn * h->ld_mod * 2));
  DFH_CHECK(dev_alloc(h->z, nn * P * ld * 2));
  DFH_CHECK(dev_alloc(h->zp, nn * P * H * 2));
  DFH_CHECK(dev_alloc(h->tvals, (size_t)(2 * RS + 64) * 4));
  h->cap_n = nn;
  h->cap_T = TT;
  h->cap_S = SS;
  h->ld_vt = ld_vt;
  return reserve_q8(h, RS > (long)SS * nn ? RS : (long)SS * nn, s);
}

// c-vector pipeline: timestep rows tv[0..R) (device floats, t then dt), condition
// and every block's adaLN modulation for rows (s, i) -> mod[(s*N + i)].
int build_modulation(DfhHandle* h, int S, int N, bool per_request_t, const float* t_dev,
                     const float* dt_dev, const TimeVals& t_host, const TimeVals& dt_host, bool has_dt,
                     const uint16_t* g, hipStream_t s) {
  const DfhConfig& c = h->cfg;
  const int H = c.hidden, fd = c.freq_dim;
  const int R = per_request_t ? N : S;  // timestep rows
  const float* freqs = P<float>(h->consts) + (c.rotary ? c.head_dim / 2 : 0);
  DFH_CHECK(timestep_embed(t_dev, t_host, R, freqs, fd / 2, fd, P<uint16_t>(h->temb_in), s));
  // time MLP: Linear(fd->H) -> SiLU -> Linear(H->H)
  DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(h->temb_in), fd, h->t_w0, h->t_b0,
                                          P<uint16_t>(h->t_hid), H, R, nullptr, H, fd), EPI_BIAS, s));
  DFH_CHECK(silu_bf16(P<uint16_t>(h->t_hid), P<uint16_t>(h->t_hid), (long)R * H, s));
  DFH_CHECK(lin(h, PC_OTHER, linear_args(P<uint16_t>(h->t_hid), H, h->t_w2, h->t_b2,
                                         P<uint16_t>(h->t_out), H, R, nullptr, H, H), EPI_BIAS, h->t2_q, s));
  const uint16_t* demb = nullptr;
  if (c.meanflow && has_dt) {
    DFH_CHECK(timestep_embed(dt_dev, dt_host, R, freqs, fd / 2, fd, P<uint16_t>(h->temb_in), s));
    DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(h->temb_in), fd, h->d_w0, h->d_b0,
                                            P<uint16_t>(h->d_hid), H, R, nullptr, H, fd), EPI_BIAS, s));
    DFH_CHECK(silu_bf16(P<uint16_t>(h->d_hid), P<uint16_t>(h->d_hid), (long)R * H, s));
    DFH_CHECK(lin(h, PC_OTHER, linear_args(P<uint16_t>(h->d_hid), H, h->d_w2, h->d_b2,
                                           P<uint16_t>(h->d_out), H, R, nullptr, H, H), EPI_BIAS, h->d2_q, s));
    demb = P<uint16_t>(h->d_out);
  }
  DFH_CHECK(condition(P<uint16_t>(h->t_out), demb, g, per_request_t ? 1 : S, N, H,
                      P<uint16_t>(h->cond), P<uint16_t>(h->cond_act), s, per_request_t));
  // every block's adaLN (and the final layer's) in one GEMM: [S*N, H] x [ld_mod, H]^T
  DFH_CHECK(lin(h, PC_OTHER, linear_args(P<uint16_t>(h->cond_act), H, h->ada_w, h->ada_b,
                                         P<uint16_t>(h->mod), h->ld_mod,
                                         (per_request_t ? 1 : S) * N, nullptr, h->ld_mod, H),
                EPI_BIAS, h->ada_q, s));
  return 0;
}

// One pass of the DiT blocks over packed rows. Input rows are in h->seq
// (before input_layer) or, with Pass::x0, already through it; the block output
// lands in h->x (h->hbuf for the latent rows of a latent tail). Row m uses modulation
// row mod_row0 + row_req[m], RoPE position row_pos[m], writes its q|k row to
// qk[l] row c_rows[m] (or m) and its V^T column vt_col[m] in vt[l].
struct Pass {
  int Mup = 0;                 // host upper bound of rows (grid sizes)
  const int* Md = nullptr;     // device row count (null: Mup rows exactly)
  long mod_row0 = 0;
  const int* row_req = nullptr;
  const int* row_pos = nullptr;
  const int* c_rows = nullptr;
  const int* vt_col = nullptr;
  std::vector<uint16_t*> qk;   // per layer
  long ldqk = 0;
  std::vector<uint16_t*> vt;   // per layer
  long ld_vt = 0;
  const AttnSeq* seqs = nullptr;
  int n_seq = 0, max_q = 0, max_kv = 0;
  bool decode = false;         // split-KV decode attention (<= 32 queries / sequence)
  float* part = nullptr;       // decode partials
  unsigned* part_cnt = nullptr;  // decode merge counters (zero between launches)
  bool kv_only_last = false;   // prefix pass: the last block only has to leave its K/V
  // input_layer rows computed before the pass (solve: the history rows once per
  // solve, the latent rows per step): block 0 reads them and writes h->x
  const uint16_t* x0 = nullptr;
  // Only the latent rows' block output is consumed (FM solve: the caller keeps
  // v[:, -P:], batched_fm.py:122-124). The last block then runs LN and the K|V
  // projection on every row (the latent queries attend over every row's K/V)
  // and the Q projection, attention, O projection, LN and MLP on the n_tail
  // latent rows alone, compacted in request order into h->hbuf (rows
  // tail_rows[j] of the pass -> row j).
  bool latent_tail = false;
  const AttnSeq* tail_seqs = nullptr;  // [n_seq]: the latent queries, output row j
  const int* tail_rows = nullptr;      // [n_tail]: pass row of compact row j
  const int* tail_req = nullptr;       // [n_tail]: request of compact row j
  const int* tail_pos = nullptr;       // [n_tail]: position of compact row j
  int n_tail = 0;
};

// The last block on the latent rows only (Pass::latent_tail), after its K|V
// GEMM over every row (q_args: that GEMM's arguments, for the latent rows' Q).
// Per row the same operations as the full block; rows that no output depends
// on are not computed.
int run_latent_tail(DfhHandle* h, const Pass& p, int l, const uint16_t* ml, long ldm, const GemmArgs& q_args,
                    const uint16_t* xin, hipStream_t s) {
  const DfhConfig& c = h->cfg;
  const int H = c.hidden, F = c.ffn, NT = p.n_tail;
  uint16_t* xl = P<uint16_t>(h->hbuf);  // compact residual rows (hbuf's LN output is consumed)
  uint16_t* hl = P<uint16_t>(h->x);     // compact LN output (x is dead once gathered; x0 is not written)
  uint16_t* al = P<uint16_t>(h->attn);  // compact attention output
  // Q of the latent rows: their LayerNorm rows compact in al, q written to their q|k rows
  DFH_CHECK(gather_rows(P<uint16_t>(h->hbuf), p.tail_rows, nullptr, NT, H, al, s));
  GemmArgs qa = q_args;
  qa.A = al; qa.lda = H; qa.B = h->qkv_w[l]; qa.ldb = H; qa.N = H; qa.col0 = 0;
  qa.M = NT; qa.M_dev = nullptr; qa.row_pos = p.tail_pos; qa.c_rows = p.tail_rows;
  DFH_CHECK(lin(h, PC_TAIL, qa, EPI_QKV, h->int8 ? h->qkv_q[l] : Q8{}, s));
  DFH_CHECK(gather_rows(xin, p.tail_rows, nullptr, NT, H, xl, s));  // the block's input rows
  prof_arm(h, PC_TAIL);
  DFH_CHECK(attention_worklist(p.tail_seqs, p.n_seq, h->attq.p, s));
  prof_arm(h, PC_TAIL);
  DFH_CHECK(seq_attention(p.qk[l], p.ldqk, p.vt[l], p.ld_vt, al, H, c.heads, h->attq.p,
                          (long)p.n_seq * ((c.patch + 127) / 128),
                          q_args.rope_q_in_attn ? q_args.rope_cos : nullptr,
                          q_args.rope_q_in_attn ? q_args.rope_sin : nullptr, s));
  GemmArgs o = linear_args(al, H, h->o_w[l], h->o_b[l], xl, H, NT, nullptr, H, H);
  o.gate = ml + 2 * H; o.ld_gate = ldm; o.row_req = p.tail_req;
  DFH_CHECK(lin(h, PC_TAIL, o, EPI_GATE_RES, h->int8 ? h->o_q[l] : Q8{}, s));
  prof_arm(h, PC_TAIL);
  DFH_CHECK(ln_modulate(xl, H, hl, H, ml + 3 * H, ml + 4 * H, ldm, p.tail_req, nullptr, NT, nullptr, H,
                        c.ln_eps, s));
  DFH_CHECK(lin(h, PC_TAIL, linear_args(hl, H, h->fc1_w[l], h->fc1_b[l], P<uint16_t>(h->ff), F, NT, nullptr,
                                        F, H), EPI_GELU, h->int8 ? h->fc1_q[l] : Q8{}, s));
  GemmArgs f2 = linear_args(P<uint16_t>(h->ff), F, h->fc2_w[l], h->fc2_b[l], xl, H, NT, nullptr, H, F);
  f2.gate = ml + 5 * H; f2.ld_gate = ldm; f2.row_req = p.tail_req;
  DFH_CHECK(lin(h, PC_TAIL, f2, EPI_GATE_RES, h->int8 ? h->fc2_q[l] : Q8{}, s));
  return 0;
}

int run_blocks(DfhHandle* h, const Pass& p, hipStream_t s) {
  const DfhConfig& c = h->cfg;
  const int H = c.hidden, F = c.ffn;
  const int Mup = p.Mup;
  const int* Md = p.Md;
  const uint16_t* mod = P<uint16_t>(h->mod) + p.mod_row0 * h->ld_mod;
  const long ldm = h->ld_mod;
  const int* row_req = p.row_req;

  // attention work list of this pass (its sequences are fixed for all blocks)
  if (!p.decode) DFH_CHECK(attention_worklist(p.seqs, p.n_seq, h->attq.p, s));
  // input_layer
  if (!p.x0)
    DFH_CHECK(lin(h, PC_OTHER, linear_args(P<uint16_t>(h->seq), H, h->in_w, h->in_b,
                                           P<uint16_t>(h->x), H, Mup, Md, H, H), EPI_BIAS, h->in_q, s,
                  tile_for(Mup, H, H, kRoleNarrow)));
  for (int l = 0; l < c.n_blocks; ++l) {
    const uint16_t* ml = mod + (long)l * 6 * H;  // shift_a, scale_a, gate_a, shift_f, scale_f, gate_f
    // block 0 of a pass with hoisted input rows reads them; its first gate-residual writes h->x
    const uint16_t* xin = (l == 0 && p.x0) ? p.x0 : P<uint16_t>(h->x);
    // the last block of a latent-tail pass also gathers bf16 LayerNorm rows
    const bool last_special = (p.latent_tail || p.kv_only_last) && l == c.n_blocks - 1;
    hipError_t lerr;
    const bool q1 = ln_q8(h, xin, P<uint16_t>(h->hbuf), ml + 0 * H, ml + 1 * H, ldm, row_req, Mup, Md,
                          h->int8 ? h->qkv_q[l] : Q8{}, last_special, s, &lerr);
    DFH_CHECK(lerr);
    GemmArgs q = linear_args(P<uint16_t>(h->hbuf), H, h->qkv_w[l], h->qkv_b[l], p.qk[l], p.ldqk, Mup, Md,
                             3 * H, H);
    q.hidden = H; q.head_dim = c.head_dim;
    q.rope_cos = c.rotary ? P<float>(h->rope_cos) : nullptr;
    q.rope_sin = c.rotary ? P<float>(h->rope_sin) : nullptr;
    q.row_pos = p.row_pos;
    // without qk-norm the stored q is the bf16 linear output the epilogue would
    // rotate, so the attention kernel rotates it (same float32 operations) once
    // per (query tile, head); split-KV decode would redo it in every key chunk
    q.rope_q_in_attn = c.rotary && c.qk_norm == 0 && !p.decode;
    const float* aq_cos = q.rope_q_in_attn ? q.rope_cos : nullptr;
    const float* aq_sin = q.rope_q_in_attn ? q.rope_sin : nullptr;
    q.qk_norm = c.qk_norm;
    q.qn_w = h->qn_w[l]; q.qn_b = h->qn_b[l]; q.kn_w = h->kn_w[l]; q.kn_b = h->kn_b[l];
    q.vt = p.vt[l]; q.ld_vt = p.ld_vt; q.vt_col = p.vt_col; q.c_rows = p.c_rows;
    if ((p.latent_tail || p.kv_only_last) && l == c.n_blocks - 1) {
      // no query of these rows is used in the last block: K|V over every row
      // (a prefix pass stops there; a latent tail projects the latent rows' Q)
      GemmArgs kv = q;
      kv.B = h->qkv_w[l] + (long)H * H; kv.N = 2 * H; kv.col0 = H;
      Q8 kv8 = h->int8 ? h->qkv_q[l] : Q8{};
      if (kv8.w) kv8.w += (long)H * H;  // scales stay indexed by the q|k|v column
      DFH_CHECK(lin(h, p.kv_only_last ? PC_QKV : PC_TAIL, kv, EPI_QKV, kv8, s, tile_for(Mup, 2 * H, H, kRoleQKV),
                    q1));
      if (p.kv_only_last) break;
      return run_latent_tail(h, p, l, ml, ldm, q, xin, s);
    }
    DFH_CHECK(lin(h, PC_QKV, q, EPI_QKV, h->int8 ? h->qkv_q[l] : Q8{}, s, tile_for(Mup, 3 * H, H, kRoleQKV), q1));
    prof_arm(h, PC_ATTN);
    if (p.decode)
      DFH_CHECK(decode_attention(p.qk[l], p.ldqk, p.vt[l], p.ld_vt, P<uint16_t>(h->attn), H, p.seqs, p.n_seq,
                                 c.heads, p.max_kv, p.part, p.part_cnt, aq_cos, aq_sin, s));
    else
      DFH_CHECK(seq_attention(p.qk[l], p.ldqk, p.vt[l], p.ld_vt, P<uint16_t>(h->attn), H, c.heads, h->attq.p,
                              (long)p.n_seq * ((p.max_q + 127) / 128), aq_cos, aq_sin, s));
    GemmArgs o = linear_args(P<uint16_t>(h->attn), H, h->o_w[l], h->o_b[l], P<uint16_t>(h->x), H,
                             Mup, Md, H, H);
    o.gate = ml + 2 * H; o.ld_gate = ldm; o.row_req = row_req;
    if (xin != P<uint16_t>(h->x)) { o.res = xin; o.ld_res = H; }
    DFH_CHECK(lin(h, PC_O, o, EPI_GATE_RES, h->int8 ? h->o_q[l] : Q8{}, s, tile_for(Mup, H, H, kRoleNarrow)));
    const bool q2 = ln_q8(h, P<uint16_t>(h->x), P<uint16_t>(h->hbuf), ml + 3 * H, ml + 4 * H, ldm, row_req, Mup,
                          Md, h->int8 ? h->fc1_q[l] : Q8{}, false, s, &lerr);
    DFH_CHECK(lerr);
    DFH_CHECK(lin(h, PC_FC1, linear_args(P<uint16_t>(h->hbuf), H, h->fc1_w[l], h->fc1_b[l],
                                         P<uint16_t>(h->ff), F, Mup, Md, F, H), EPI_GELU,
                  h->int8 ? h->fc1_q[l] : Q8{}, s, tile_for(Mup, F, H, kRoleWide), q2));
    GemmArgs f2 = linear_args(P<uint16_t>(h->ff), F, h->fc2_w[l], h->fc2_b[l], P<uint16_t>(h->x), H,
                              Mup, Md, H, F);
    f2.gate = ml + 5 * H; f2.ld_gate = ldm; f2.row_req = row_req;
    DFH_CHECK(lin(h, PC_FC2, f2, EPI_GATE_RES, h->int8 ? h->fc2_q[l] : Q8{}, s, tile_for(Mup, H, F, kRoleNarrow)));
  }
  return 0;
}

// The FM pass over the packed requests of layout(): rows m of h->seq, request
// row_req[m], q|k into the workspace, V^T in h->vt.
int dit_blocks(DfhHandle* h, int n, int T, long mod_row0, hipStream_t s, bool latent_tail = false,
               const uint16_t* x0 = nullptr) {
  const DfhConfig& c = h->cfg;
  Pass p;
  p.Mup = n * T;
  p.Md = P<int>(h->counts);
  p.mod_row0 = mod_row0;
  p.row_req = P<int>(h->row_req);
  p.row_pos = P<int>(h->row_pos);
  p.vt_col = P<int>(h->vt_col);
  p.qk.assign(c.n_blocks, P<uint16_t>(h->qk));
  p.ldqk = qk_stride(c);
  p.vt.assign(c.n_blocks, P<uint16_t>(h->vt));
  p.ld_vt = h->ld_vt;
  p.seqs = P<AttnSeq>(h->seqs);
  p.n_seq = n;
  p.max_q = T;
  p.x0 = x0;
  if (latent_tail) {
    p.latent_tail = true;
    p.tail_seqs = P<AttnSeq>(h->tail_seqs);
    p.tail_rows = P<int>(h->patch_rows);
    p.tail_req = P<int>(h->tail_req);
    p.tail_pos = P<int>(h->tail_pos);
    p.n_tail = n * c.patch;
  }
  return run_blocks(h, p, s);
}

// Packed layout of n requests, T = max history + P. Padded inputs: pos_ids and
// inp [n, T, H]. Varlen inputs: lens [n] and the history bases src_rows [n].
int layout(DfhHandle* h, int n, int T, const void* pos_ids, const void* inp, hipStream_t s,
           const int* lens = nullptr, const uint16_t* const* src_rows = nullptr, long src_stride = 0) {
  const DfhConfig& c = h->cfg;
  DFH_CHECK(fm_layout(reinterpret_cast<const float*>(pos_ids), lens, n, T, c.patch, P<int>(h->cu_rows),
                      P<int>(h->cu_vt), P<int>(h->hist_len), P<int>(h->counts), P<int>(h->err),
                      P<AttnSeq>(h->seqs), P<AttnSeq>(h->tail_seqs), P<int>(h->tail_req), P<int>(h->tail_pos),
                      s));
  DFH_CHECK(fm_gather(reinterpret_cast<const uint16_t*>(inp), src_rows, src_stride, n, T, c.patch, c.hidden,
                      P<int>(h->cu_rows), P<int>(h->cu_vt), P<int>(h->hist_len), P<uint16_t>(h->seq),
                      P<int>(h->row_req), P<int>(h->row_pos), P<int>(h->vt_col),
                      P<int>(h->patch_rows), P<int>(h->err), s));
  if (c.rotary)
    DFH_CHECK(rope_table(P<float>(h->consts), c.head_dim / 2, T, P<float>(h->rope_cos),
                         P<float>(h->rope_sin), s));
  return 0;
}

// The NFE steps of one MeanFlow solve on the packed layout built by layout().
int solve_steps(DfhHandle* h, int n, int T, int S, const void* g_cond, const void* noise, void* out,
                const float* t_grid, const float* dt_grid, hipStream_t s) {
  const DfhConfig& c = h->cfg;
  const int H = c.hidden, Pp = c.patch, ld = c.latent_dim;
  // timestep rows t_0..t_{S-1} and dt_0..dt_{S-1} travel as kernel arguments
  TimeVals tv{}, dtv{};
  for (int k = 0; k < S; ++k) { tv.v[k] = t_grid[k]; dtv.v[k] = dt_grid[k]; }
  if (build_modulation(h, S, n, false, nullptr, nullptr, tv, dtv, true,
                       reinterpret_cast<const uint16_t*>(g_cond), s))
    return 1;
  DFH_CHECK(hipMemcpyAsync(h->z.p, noise, (size_t)n * Pp * ld * 2, hipMemcpyDeviceToDevice, s));
  const int NP = n * Pp;
  // input_layer of every packed row once: a history row's does not depend on the
  // step (no t or z); the latent rows' are replaced every step
  DFH_CHECK(lin(h, PC_OTHER, linear_args(P<uint16_t>(h->seq), H, h->in_w, h->in_b, P<uint16_t>(h->x0), H,
                                         n * T, P<int>(h->counts), H, H), EPI_BIAS, h->in_q, s,
                tile_for(n * T, H, H, kRoleNarrow)));
  for (int st = 0; st < S; ++st) {
    // zp = coordinate_proj(z); its input_layer rows -> the latent rows of x0
    DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(h->z), ld, h->coord_w, h->coord_b,
                                            P<uint16_t>(h->zp), H, NP, nullptr, H, ld), EPI_BIAS, s));
    DFH_CHECK(lin(h, PC_OTHER, linear_args(P<uint16_t>(h->zp), H, h->in_w, h->in_b, P<uint16_t>(h->fin), H,
                                           NP, nullptr, H, H), EPI_BIAS, h->in_q, s));
    DFH_CHECK(scatter_rows(P<uint16_t>(h->fin), P<int>(h->patch_rows), NP, H, P<uint16_t>(h->x0), s));
    const bool tail = h->latent_tail;
    if (dit_blocks(h, n, T, (long)st * n, s, tail, P<uint16_t>(h->x0))) return 1;
    // FinalLayer on the latent rows only (compact in h->hbuf after a latent tail)
    const uint16_t* mf = P<uint16_t>(h->mod) + (long)st * n * h->ld_mod + (long)c.n_blocks * 6 * H;
    prof_arm(h, tail ? PC_TAIL : PC_LN);
    if (tail)
      DFH_CHECK(ln_modulate(P<uint16_t>(h->hbuf), H, P<uint16_t>(h->fin), H, mf, mf + H, h->ld_mod,
                            P<int>(h->tail_req), nullptr, NP, nullptr, H, c.ln_eps, s));
    else
      DFH_CHECK(ln_modulate(P<uint16_t>(h->x), H, P<uint16_t>(h->fin), H, mf, mf + H, h->ld_mod,
                            P<int>(h->row_req), P<int>(h->patch_rows), NP, nullptr, H, c.ln_eps, s));
    DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(h->fin), H, h->fin_w, h->fin_b,
                                            P<uint16_t>(h->vel), ld, NP, nullptr, ld, H), EPI_BIAS, s));
    DFH_CHECK(z_update(P<uint16_t>(h->z), P<uint16_t>(h->vel), dt_grid[st], (long)NP * ld, s));
  }
  DFH_CHECK(hipMemcpyAsync(out, h->z.p, (size_t)NP * ld * 2, hipMemcpyDeviceToDevice, s));
  return 0;
}

}  // namespace

extern "C" {

const char* dfh_last_error(void) { return g_err.c_str(); }

int dfh_create(const DfhConfig* cfg, DfhHandle** out) {
  if (!cfg || !out) return fail("null argument");
  if (check_cfg(*cfg)) return 1;
  DfhHandle* h = new DfhHandle();
  h->cfg = *cfg;
  if (cfg->rotary) h->rope_inv_freq.assign(cfg->rope_inv_freq, cfg->rope_inv_freq + cfg->head_dim / 2);
  h->temb_freqs.assign(cfg->temb_freqs, cfg->temb_freqs + cfg->freq_dim / 2);
  h->cfg.rope_inv_freq = nullptr;
  h->cfg.temb_freqs = nullptr;
  h->ld_mod = cfg->n_blocks * 6 * cfg->hidden + 2 * cfg->hidden;
  std::vector<float> consts(h->rope_inv_freq);
  consts.insert(consts.end(), h->temb_freqs.begin(), h->temb_freqs.end());
  hipError_t e = dev_alloc(h->consts, consts.size() * 4);
  if (e == hipSuccess) e = hipMemcpy(h->consts.p, consts.data(), consts.size() * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    delete h;
    return fail("dfh_create: %s", hipGetErrorString(e));
  }
  *out = h;
  return 0;
}

int dfh_destroy(DfhHandle* h) {
  if (!h) return 0;
  (void)hipDeviceSynchronize();
  DevBuf* bufs[] = {&h->w_arena, &h->consts, &h->seq, &h->x, &h->hbuf, &h->qk, &h->attn, &h->ff,
                    &h->vt, &h->row_req, &h->row_pos, &h->vt_col, &h->cu_rows, &h->cu_vt,
                    &h->hist_len, &h->counts, &h->err, &h->patch_rows, &h->seqs, &h->rope_cos, &h->rope_sin,
                    &h->temb_in, &h->t_hid, &h->t_out, &h->d_hid, &h->d_out, &h->cond,
                    &h->cond_act, &h->mod, &h->z, &h->zp, &h->fin, &h->vel, &h->tvals, &h->splitws, &h->attq,
                    &h->x0, &h->tail_seqs, &h->tail_req, &h->tail_pos, &h->w8, &h->aq, &h->asx};
  for (DevBuf* b : bufs)
    if (b->p) (void)hipFree(b->p);
  for (hipEvent_t ev : h->ev_pool) (void)hipEventDestroy(ev);
  delete h;
  return 0;
}

int dfh_set_weights(DfhHandle* h, const DfhWeights* w, void* stream) {
  if (h) h->int8 = false;  // the int8 weights were made from the previous weights
  if (!h || !w || !w->blocks) return fail("null argument");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const DfhConfig& c = h->cfg;
  const long H = c.hidden, F = c.ffn, ld = c.latent_dim, fd = c.freq_dim, hd = c.head_dim;
  const int nb = c.n_blocks;
  if (!w->input_w || !w->input_b || !w->t_w0 || !w->t_b0 || !w->t_w2 || !w->t_b2 || !w->final_ada_w ||
      !w->final_ada_b || !w->final_w || !w->final_b || !w->coord_w || !w->coord_b)
    return fail("dfh_set_weights: a required tensor is NULL");
  if (c.meanflow && (!w->d_w0 || !w->d_b0 || !w->d_w2 || !w->d_b2))
    return fail("dfh_set_weights: meanflow DiT needs the duration embedder");
  // arena layout (elements); every piece 256-B aligned
  struct Piece { const void* src; long elems; const uint16_t** dst; };
  std::vector<Piece> pieces;
  std::vector<std::pair<long, long>> zero_fill;  // (offset, elems) for absent biases
  long off = 0;
  auto take = [&](long elems) { long o = off; off += (elems + 127) / 128 * 128; return o; };
  std::vector<long> offs;
  struct Copy { const void* src; long dst_off; long elems; };
  std::vector<Copy> copies;
  auto add = [&](const void* src, long elems) -> long {
    long o = take(elems);
    if (src) copies.push_back({src, o, elems});
    else zero_fill.push_back({o, elems});
    return o;
  };
  const long o_in_w = add(w->input_w, H * H), o_in_b = add(w->input_b, H);
  const long o_t_w0 = add(w->t_w0, H * fd), o_t_b0 = add(w->t_b0, H);
  const long o_t_w2 = add(w->t_w2, H * H), o_t_b2 = add(w->t_b2, H);
  long o_d_w0 = 0, o_d_b0 = 0, o_d_w2 = 0, o_d_b2 = 0;
  if (c.meanflow) {
    o_d_w0 = add(w->d_w0, H * fd); o_d_b0 = add(w->d_b0, H);
    o_d_w2 = add(w->d_w2, H * H); o_d_b2 = add(w->d_b2, H);
  }
  // all adaLN rows contiguous: blocks 0..nb-1 (6H each) then the final layer (2H)
  const long o_ada_w = take((long)h->ld_mod * H);
  const long o_ada_b = take(h->ld_mod);
  for (int l = 0; l < nb; ++l) {
    const DfhBlockWeights& b = w->blocks[l];
    if (!b.ada_w || !b.ada_b) return fail("block %d: adaLN weights missing", l);
    copies.push_back({b.ada_w, o_ada_w + (long)l * 6 * H * H, 6 * H * H});
    copies.push_back({b.ada_b, o_ada_b + (long)l * 6 * H, 6 * H});
  }
  copies.push_back({w->final_ada_w, o_ada_w + (long)nb * 6 * H * H, 2 * H * H});
  copies.push_back({w->final_ada_b, o_ada_b + (long)nb * 6 * H, 2 * H});
  const long o_fin_w = add(w->final_w, ld * H), o_fin_b = add(w->final_b, ld);
  const long o_co_w = add(w->coord_w, H * ld), o_co_b = add(w->coord_b, H);
  std::vector<long> o_qkv_w(nb), o_qkv_b(nb), o_o_w(nb), o_o_b(nb), o_f1w(nb), o_f1b(nb), o_f2w(nb),
      o_f2b(nb), o_qn_w(nb), o_qn_b(nb), o_kn_w(nb), o_kn_b(nb);
  for (int l = 0; l < nb; ++l) {
    const DfhBlockWeights& b = w->blocks[l];
    if (!b.q_w || !b.k_w || !b.v_w || !b.o_w || !b.o_b || !b.fc1_w || !b.fc1_b || !b.fc2_w || !b.fc2_b)
      return fail("block %d: a required tensor is NULL", l);
    o_qkv_w[l] = take(3 * H * H);
    copies.push_back({b.q_w, o_qkv_w[l], H * H});
    copies.push_back({b.k_w, o_qkv_w[l] + H * H, H * H});
    copies.push_back({b.v_w, o_qkv_w[l] + 2 * H * H, H * H});
    o_qkv_b[l] = -1;
    if (c.qkv_bias) {
      if (!b.q_b || !b.k_b || !b.v_b) return fail("block %d: qkv_bias set but a bias is NULL", l);
      o_qkv_b[l] = take(3 * H);
      copies.push_back({b.q_b, o_qkv_b[l], H});
      copies.push_back({b.k_b, o_qkv_b[l] + H, H});
      copies.push_back({b.v_b, o_qkv_b[l] + 2 * H, H});
    }
    o_o_w[l] = add(b.o_w, H * H); o_o_b[l] = add(b.o_b, H);
    o_f1w[l] = add(b.fc1_w, F * H); o_f1b[l] = add(b.fc1_b, F);
    o_f2w[l] = add(b.fc2_w, H * F); o_f2b[l] = add(b.fc2_b, H);
    o_qn_w[l] = o_qn_b[l] = o_kn_w[l] = o_kn_b[l] = -1;
    if (c.qk_norm) {
      if (!b.q_norm_w || !b.k_norm_w) return fail("block %d: qk_norm weights missing", l);
      o_qn_w[l] = add(b.q_norm_w, hd); o_kn_w[l] = add(b.k_norm_w, hd);
      if (c.qk_norm == 1) {
        if (!b.q_norm_b || !b.k_norm_b) return fail("block %d: qk LayerNorm biases missing", l);
        o_qn_b[l] = add(b.q_norm_b, hd); o_kn_b[l] = add(b.k_norm_b, hd);
      }
    }
  }
  DFH_CHECK(hipStreamSynchronize(s));
  DFH_CHECK(dev_alloc(h->w_arena, (size_t)off * 2));
  uint16_t* base = P<uint16_t>(h->w_arena);
  for (const Copy& cp : copies)
    DFH_CHECK(hipMemcpyAsync(base + cp.dst_off, cp.src, cp.elems * 2, hipMemcpyDeviceToDevice, s));
  for (auto& z : zero_fill) DFH_CHECK(hipMemsetAsync(base + z.first, 0, z.second * 2, s));
  DFH_CHECK(hipStreamSynchronize(s));
  auto at = [&](long o) -> const uint16_t* { return o < 0 ? nullptr : base + o; };
  h->in_w = at(o_in_w); h->in_b = at(o_in_b);
  h->t_w0 = at(o_t_w0); h->t_b0 = at(o_t_b0); h->t_w2 = at(o_t_w2); h->t_b2 = at(o_t_b2);
  if (c.meanflow) {
    h->d_w0 = at(o_d_w0); h->d_b0 = at(o_d_b0); h->d_w2 = at(o_d_w2); h->d_b2 = at(o_d_b2);
  } else {
    h->d_w0 = h->d_b0 = h->d_w2 = h->d_b2 = nullptr;
  }
  h->ada_w = at(o_ada_w); h->ada_b = at(o_ada_b);
  h->fin_w = at(o_fin_w); h->fin_b = at(o_fin_b);
  h->coord_w = at(o_co_w); h->coord_b = at(o_co_b);
  h->qkv_w.resize(nb); h->qkv_b.resize(nb); h->o_w.resize(nb); h->o_b.resize(nb);
  h->fc1_w.resize(nb); h->fc1_b.resize(nb); h->fc2_w.resize(nb); h->fc2_b.resize(nb);
  h->qn_w.resize(nb); h->qn_b.resize(nb); h->kn_w.resize(nb); h->kn_b.resize(nb);
  for (int l = 0; l < nb; ++l) {
    h->qkv_w[l] = at(o_qkv_w[l]); h->qkv_b[l] = at(o_qkv_b[l]);
    h->o_w[l] = at(o_o_w[l]); h->o_b[l] = at(o_o_b[l]);
    h->fc1_w[l] = at(o_f1w[l]); h->fc1_b[l] = at(o_f1b[l]);
    h->fc2_w[l] = at(o_f2w[l]); h->fc2_b[l] = at(o_f2b[l]);
    h->qn_w[l] = at(o_qn_w[l]); h->qn_b[l] = at(o_qn_b[l]);
    h->kn_w[l] = at(o_kn_w[l]); h->kn_b[l] = at(o_kn_b[l]);
  }
  h->weights_set = true;
  return 0;
}

// W8A8 mode of the solve and forward (the reference's quantize_dit_ on the DiT,
// int8_dit.py:34-85): the int8 weights come from the caller or are quantised
// here from the handle's bf16 weights, as Int8DynamicLinear(lin) does.
int dfh_set_int8(DfhHandle* h, int enable, const DfhInt8Weights* w, void* stream) {
  if (!h) return fail("dfh_set_int8: NULL handle");
  if (!enable) {
    h->int8 = false;
    return 0;
  }
  if (!h->weights_set) return fail("dfh_set_int8: set the weights first");
  const DfhConfig& c = h->cfg;
  const long H = c.hidden, F = c.ffn;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  struct Item {
    const uint16_t* src;      // bf16 [N, K]
    DfhInt8Linear given;      // caller's int8 weight (NULL: quantise src)
    long N, K;
    Q8* dst;
  };
  std::vector<Item> items;
  auto given = [&](const DfhInt8Linear* a) { return a ? *a : DfhInt8Linear{nullptr, nullptr}; };
  h->qkv_q.assign(c.n_blocks, Q8{});
  h->o_q.assign(c.n_blocks, Q8{});
  h->fc1_q.assign(c.n_blocks, Q8{});
  h->fc2_q.assign(c.n_blocks, Q8{});
  h->d2_q = Q8{};
  items.push_back({h->in_w, given(w ? &w->input : nullptr), H, H, &h->in_q});
  items.push_back({h->t_w2, given(w ? &w->t_mlp2 : nullptr), H, H, &h->t2_q});
  if (c.meanflow) items.push_back({h->d_w2, given(w ? &w->d_mlp2 : nullptr), H, H, &h->d2_q});
  items.push_back({h->ada_w, given(w ? &w->ada : nullptr), h->ld_mod, H, &h->ada_q});
  for (int l = 0; l < c.n_blocks; ++l) {
    items.push_back({h->qkv_w[l], given(w && w->qkv ? &w->qkv[l] : nullptr), 3 * H, H, &h->qkv_q[l]});
    items.push_back({h->o_w[l], given(w && w->o ? &w->o[l] : nullptr), H, H, &h->o_q[l]});
    items.push_back({h->fc1_w[l], given(w && w->fc1 ? &w->fc1[l] : nullptr), F, H, &h->fc1_q[l]});
    items.push_back({h->fc2_w[l], given(w && w->fc2 ? &w->fc2[l] : nullptr), H, F, &h->fc2_q[l]});
  }
  long total = 0;
  std::vector<long> wo, so;
  for (auto& it : items) {
    if ((it.given.w == nullptr) != (it.given.scale == nullptr))
      return fail("dfh_set_int8: an int8 weight needs both its values and its scales");
    wo.push_back(total);
    total = (total + it.N * it.K + 255) / 256 * 256;
    so.push_back(total);
    total = (total + it.N * 4 + 255) / 256 * 256;
  }
  DFH_CHECK(hipStreamSynchronize(s));
  h->int8 = false;
  DFH_CHECK(dev_alloc(h->w8, total));
  for (size_t i = 0; i < items.size(); ++i) {
    Item& it = items[i];
    int8_t* q = P<int8_t>(h->w8) + wo[i];
    float* sc = reinterpret_cast<float*>(P<char>(h->w8) + so[i]);
    if (it.given.w) {
      DFH_CHECK(hipMemcpyAsync(q, it.given.w, it.N * it.K, hipMemcpyDeviceToDevice, s));
      DFH_CHECK(hipMemcpyAsync(sc, it.given.scale, it.N * 4, hipMemcpyDeviceToDevice, s));
    } else {
      DFH_CHECK(quant_weight_f32(it.src, q, sc, (int)it.N, (int)it.K, s));
    }
    *it.dst = Q8{q, sc};
  }
  h->int8 = true;
  const long rows = h->cap_M > (long)h->cap_S * h->cap_n ? h->cap_M : (long)h->cap_S * h->cap_n;
  if (reserve_q8(h, rows > 0 ? rows : 1, s)) return 1;
  DFH_CHECK(hipStreamSynchronize(s));
  return 0;
}

int dfh_reserve(DfhHandle* h, int n, int T, int S, void* stream) {
  if (!h) return fail("null handle");
  if (n <= 0 || n > 1024 || T <= h->cfg.patch || S <= 0 || S > 16)
    return fail("dfh_reserve: bad shape n=%d T=%d steps=%d", n, T, S);
  return reserve(h, n, T, S, reinterpret_cast<hipStream_t>(stream));
}

int dfh_meanflow_solve(DfhHandle* h, const DfhSolveArgs* a, void* stream) {
  if (!h || !a) return fail("null argument");
  if (!h->weights_set) return fail("dfh_meanflow_solve: weights not set");
  const DfhConfig& c = h->cfg;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int n = a->n, T = a->total_len, S = a->num_steps;
  if (n <= 0 || n > 1024 || T <= c.patch || S <= 0 || S > 16)
    return fail("dfh_meanflow_solve: bad shape n=%d T=%d steps=%d", n, T, S);
  if (!a->input_sequence || !a->pos_ids || !a->noise || !a->out || !a->t_grid || !a->dt_grid)
    return fail("dfh_meanflow_solve: a required pointer is NULL");
  if (!c.meanflow) return fail("dfh_meanflow_solve: DiT has no duration embedder (not MeanFlow)");
  if ((long)n * T * (c.ffn > qk_stride(c) ? c.ffn : qk_stride(c)) >= (1L << 31))
    return fail("dfh_meanflow_solve: n*T too large for 32-bit offsets");
  if (reserve(h, n, T, S, s)) return 1;
  if (layout(h, n, T, a->pos_ids, a->input_sequence, s)) return 1;
  return solve_steps(h, n, T, S, a->g_cond, a->noise, a->out, a->t_grid, a->dt_grid, s);
}

int dfh_meanflow_solve_varlen(DfhHandle* h, const DfhVarlenSolveArgs* a, void* stream) {
  if (!h || !a) return fail("null argument");
  if (!h->weights_set) return fail("dfh_meanflow_solve_varlen: weights not set");
  const DfhConfig& c = h->cfg;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int n = a->n, S = a->num_steps;
  if (n <= 0 || n > 1024 || a->max_hist <= 0 || S <= 0 || S > 16)
    return fail("dfh_meanflow_solve_varlen: bad shape n=%d max_hist=%d steps=%d", n, a->max_hist, S);
  if (!a->hist_rows || !a->hist_len || !a->noise || !a->out || !a->t_grid || !a->dt_grid)
    return fail("dfh_meanflow_solve_varlen: a required pointer is NULL");
  if (a->row_stride < c.hidden || a->row_stride % 8 != 0)
    return fail("dfh_meanflow_solve_varlen: row_stride %ld must be >= hidden and a multiple of 8",
                a->row_stride);
  if (!c.meanflow) return fail("dfh_meanflow_solve_varlen: DiT has no duration embedder (not MeanFlow)");
  const int T = a->max_hist + c.patch;
  if ((long)n * T * (c.ffn > qk_stride(c) ? c.ffn : qk_stride(c)) >= (1L << 31))
    return fail("dfh_meanflow_solve_varlen: n*T too large for 32-bit offsets");
  if (reserve(h, n, T, S, s)) return 1;
  if (layout(h, n, T, nullptr, nullptr, s, a->hist_len,
             reinterpret_cast<const uint16_t* const*>(a->hist_rows), a->row_stride))
    return 1;
  return solve_steps(h, n, T, S, a->g_cond, a->noise, a->out, a->t_grid, a->dt_grid, s);
}

int dfh_dit_forward(DfhHandle* h, const DfhForwardArgs* a, void* stream) {
  if (!h || !a) return fail("null argument");
  if (!h->weights_set) return fail("dfh_dit_forward: weights not set");
  const DfhConfig& c = h->cfg;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int n = a->n, T = a->total_len;
  if (n <= 0 || n > 1024 || T <= c.patch) return fail("dfh_dit_forward: bad shape n=%d T=%d", n, T);
  if (!a->x || !a->timesteps || !a->pos_ids || !a->out) return fail("dfh_dit_forward: NULL pointer");
  if ((long)n * T * (c.ffn > qk_stride(c) ? c.ffn : qk_stride(c)) >= (1L << 31)) return fail("dfh_dit_forward: n*T too large");
  if (reserve(h, n, T, 1, s)) return 1;
  const int H = c.hidden, Pp = c.patch, ld = c.latent_dim;
  if (layout(h, n, T, a->pos_ids, a->x, s)) return 1;
  TimeVals none{};
  const bool has_dt = c.meanflow && a->duration != nullptr;
  if (build_modulation(h, 1, n, true, reinterpret_cast<const float*>(a->timesteps),
                       reinterpret_cast<const float*>(a->duration), none, none, has_dt,
                       reinterpret_cast<const uint16_t*>(a->g_cond), s))
    return 1;
  if (dit_blocks(h, n, T, 0, s)) return 1;
  // FinalLayer on every packed row, then scatter back to the padded layout
  const int Mup = n * T;
  const uint16_t* mf = P<uint16_t>(h->mod) + (long)c.n_blocks * 6 * H;
  DFH_CHECK(ln_modulate(P<uint16_t>(h->x), H, P<uint16_t>(h->fin), H, mf, mf + H, h->ld_mod,
                        P<int>(h->row_req), nullptr, Mup, P<int>(h->counts), H, c.ln_eps, s));
  DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(h->fin), H, h->fin_w, h->fin_b,
                                          P<uint16_t>(h->vel), ld, Mup, P<int>(h->counts), ld, H),
                 EPI_BIAS, s));
  DFH_CHECK(dfh::unpack_rows(P<uint16_t>(h->vel), n, T, Pp, ld, P<int>(h->cu_rows), P<int>(h->hist_len),
                             reinterpret_cast<uint16_t*>(a->out), s));
  return 0;
}

int dfh_input_status(DfhHandle* h, int* flags, void* stream) {
  if (!h || !flags) return fail("null argument");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  *flags = 0;
  if (!h->err.p) return 0;
  DFH_CHECK(hipMemcpyAsync(flags, h->err.p, 4, hipMemcpyDeviceToHost, s));
  DFH_CHECK(hipStreamSynchronize(s));
  DFH_CHECK(hipMemsetAsync(h->err.p, 0, 4, s));
  DFH_CHECK(hipStreamSynchronize(s));
  return 0;
}

int dfh_set_ksplit(DfhHandle* h, int enable) {
  if (!h) return fail("null handle");
  h->ksplit = enable != 0;
  return 0;
}

int dfh_set_ln_quant(DfhHandle* h, int enable) {
  if (!h) return fail("null handle");
  h->ln_quant = enable != 0;
  return 0;
}

int dfh_set_latent_tail(DfhHandle* h, int enable) {
  if (!h) return fail("null handle");
  h->latent_tail = enable != 0;
  return 0;
}

int dfh_profile_enable(DfhHandle* h, int enable) {
  if (!h) return fail("null handle");
  if (enable && h->ev_pool.empty()) {
    h->ev_pool.resize(1 << 14);
    for (auto& ev : h->ev_pool) DFH_CHECK(hipEventCreate(&ev));
  }
  h->prof = enable != 0;
  return 0;
}

int dfh_profile_classes(DfhHandle* h, unsigned mask, int every) {
  if (!h) return fail("null handle");
  if (every < 1) return fail("every must be at least 1 (got %d)", every);
  h->prof_mask = mask;
  h->prof_every = every;
  for (auto& n : h->prof_seen) n = 0;
  return 0;
}

int dfh_profile_read(DfhHandle* h, double* ms, long* cnt, int n_classes) {
  if (!h) return fail("null handle");
  for (auto& u : h->ev_used) {
    DFH_CHECK(hipEventSynchronize(h->ev_pool[u.second + 1]));
    float t = 0.f;
    DFH_CHECK(hipEventElapsedTime(&t, h->ev_pool[u.second], h->ev_pool[u.second + 1]));
    h->prof_ms[u.first] += t;
    h->prof_n[u.first] += 1;
  }
  h->ev_used.clear();
  h->ev_next = 0;
  for (int i = 0; i < n_classes && i < PC_N; ++i) {
    if (ms) ms[i] = h->prof_ms[i];
    if (cnt) cnt[i] = h->prof_n[i];
    h->prof_ms[i] = 0;
    h->prof_n[i] = 0;
  }
  return 0;
}

int dfh_gemm_bf16(const void* A, long lda, const void* B, long ldb, void* C, long ldc, const void* bias,
                  int M, int N, int K, int epilogue, int tile, void* stream) {
  return dfh_gemm_bf16_ws(A, lda, B, ldb, C, ldc, bias, M, N, K, epilogue, tile, nullptr, 0, stream);
}

int dfh_gemm_bf16_ws(const void* A, long lda, const void* B, long ldb, void* C, long ldc, const void* bias,
                     int M, int N, int K, int epilogue, int tile, void* ws, long ws_bytes, void* stream) {
  if (!A || !B || !C) return fail("dfh_gemm_bf16: NULL pointer");
  if (epilogue != EPI_BIAS && epilogue != EPI_GELU && epilogue != EPI_SILU && epilogue != EPI_F32)
    return fail("dfh_gemm_bf16: epilogue %d not exposed", epilogue);
  if (lda % 8 || ldb % 8 || ldc % 8 || lda < K || ldb < K || ldc < N)
    return fail("dfh_gemm_bf16: leading dimensions must be >= the row length and multiples of 8");
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = reinterpret_cast<const uint16_t*>(A); a.lda = lda;
  a.B = reinterpret_cast<const uint16_t*>(B); a.ldb = ldb;
  a.C = reinterpret_cast<uint16_t*>(C); a.Cf = reinterpret_cast<float*>(C); a.ldc = ldc;
  a.bias = reinterpret_cast<const uint16_t*>(bias);
  a.M = M; a.N = N; a.K = K;
  a.ws = reinterpret_cast<float*>(ws); a.ws_elems = ws ? ws_bytes / 4 : 0;
  hipError_t e = gemm_bf16(a, epilogue, reinterpret_cast<hipStream_t>(stream), tile);
  if (e != hipSuccess) return fail("dfh_gemm_bf16(M=%d N=%d K=%d tile=%d): %s", M, N, K, tile,
                                   hipGetErrorString(e));
  return 0;
}

int dfh_store_kvcache(const void* key, long key_stride, const void* value, long value_stride, void* k_cache,
                      void* v_cache, const int* slot_mapping, int n_tokens, int D, void* stream) {
  if (n_tokens < 0 || D <= 0) return fail("dfh_store_kvcache: bad shape n=%d D=%d", n_tokens, D);
  if (n_tokens == 0) return 0;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return fail("dfh_store_kvcache: NULL pointer");
  if (D % 8 || key_stride % 8 || value_stride % 8 || key_stride < D || value_stride < D)
    return fail("dfh_store_kvcache: D and strides must be multiples of 8 (strides >= D)");
  if (((uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15)
    return fail("dfh_store_kvcache: buffers must be 16-byte aligned");
  DFH_CHECK(dfh::store_kvcache(static_cast<const uint16_t*>(key), key_stride, static_cast<const uint16_t*>(value),
                               value_stride, static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                               slot_mapping, n_tokens, D, reinterpret_cast<hipStream_t>(stream)));
  return 0;
}

long dfh_paged_attention_workspace(const DfhPagedAttnArgs* a) {
  if (!a || a->batch <= 0 || a->num_kv_heads <= 0 || a->num_heads % a->num_kv_heads || a->max_seqlen_q <= 0 ||
      a->max_seqlen_k <= 0)
    return 0;
  return dfh::paged_attention_ws_bytes(a->batch, a->num_kv_heads, a->num_heads / a->num_kv_heads, a->max_seqlen_q,
                                      a->max_seqlen_k, a->head_dim, a->total_q > 0 ? a->total_q : 0);
}

int dfh_paged_attention(const DfhPagedAttnArgs* a, void* stream) {
  if (!a) return fail("null argument");
  if (a->batch <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->num_heads % a->num_kv_heads)
    return fail("dfh_paged_attention: bad heads (batch=%d heads=%d kv_heads=%d)", a->batch, a->num_heads,
                a->num_kv_heads);
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail("dfh_paged_attention: head_dim %d not supported (64 or 128)", a->head_dim);
  if (a->max_seqlen_q <= 0 || a->max_seqlen_k <= 0)
    return fail("dfh_paged_attention: max_seqlen_q / max_seqlen_k must be positive");
  if (!a->q || !a->k || !a->v || !a->out || !a->cu_seqlens_q || !a->workspace)
    return fail("dfh_paged_attention: a required pointer is NULL");
  if (!a->cu_seqlens_k && !(a->seqlens_k && a->block_table))
    return fail("dfh_paged_attention: key lengths need cu_seqlens_k (or seqlens_k with a block table)");
  if (a->block_table && (a->block_size <= 0 || a->block_size % 256 || a->block_table_stride <= 0))
    return fail("dfh_paged_attention: block_size %d must be a positive multiple of 256", a->block_size);
  const long D = (long)a->num_kv_heads * a->head_dim;
  if (a->q_stride < (long)a->num_heads * a->head_dim || a->kv_stride < D || a->q_stride % 8 || a->kv_stride % 8 ||
      a->out_stride < (long)a->num_heads * a->head_dim)
    return fail("dfh_paged_attention: bad strides");
  if (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->v) & 15)
    return fail("dfh_paged_attention: q, k, v must be 16-byte aligned");
  if ((uintptr_t)a->workspace & 15) return fail("dfh_paged_attention: workspace must be 16-byte aligned");
  const long need = dfh_paged_attention_workspace(a);
  if (a->workspace_bytes < need)
    return fail("dfh_paged_attention: workspace %ld bytes < %ld needed", a->workspace_bytes, need);
  dfh::PagedAttnArgs x{};
  x.batch = a->batch; x.heads = a->num_heads; x.kv_heads = a->num_kv_heads; x.head_dim = a->head_dim;
  x.max_q = a->max_seqlen_q; x.max_k = a->max_seqlen_k;
  x.q = static_cast<const uint16_t*>(a->q); x.q_stride = a->q_stride; x.cu_q = a->cu_seqlens_q;
  x.k = static_cast<const uint16_t*>(a->k); x.v = static_cast<const uint16_t*>(a->v); x.kv_stride = a->kv_stride;
  x.cu_k = a->cu_seqlens_k; x.seqlens_k = a->seqlens_k;
  x.block_table = a->block_table; x.bt_stride = a->block_table_stride; x.block_size = a->block_size;
  x.out = static_cast<uint16_t*>(a->out); x.out_stride = a->out_stride;
  x.scale = a->softmax_scale; x.causal = a->causal;
  x.ws = a->workspace;
  x.total_q = a->total_q > 0 ? a->total_q : 0;
  DFH_CHECK(dfh::paged_attention(x, reinterpret_cast<hipStream_t>(stream)));
  return 0;
}

int dfh_paged_attention_noalloc(const DfhPagedAttnArgs* a, void* stream) {
  if (!a) return fail("null argument");
  const long need = dfh_paged_attention_workspace(a);
  if (need > dfh::kPagedScratchBytes)
    return fail("dfh_paged_attention_noalloc: this call needs %ld bytes of workspace, more than the %ld-byte static "
                "scratch (use dfh_paged_attention with a workspace)", need, dfh::kPagedScratchBytes);
  hipError_t e = hipSuccess;
  void* ws = dfh::paged_scratch(&e);
  if (!ws) return fail("dfh_paged_attention_noalloc: scratch address: %s", hipGetErrorString(e));
  DfhPagedAttnArgs b = *a;
  b.workspace = ws;
  b.workspace_bytes = dfh::kPagedScratchBytes;
  return dfh_paged_attention(&b, stream);
}

int dfh_quant_act_i8(const void* x, long ldx, void* q, long ldq, void* scale, int M, int K, void* stream) {
  if (!x || !q || !scale) return fail("dfh_quant_act_i8: NULL pointer");
  if (M < 0 || K <= 0 || K % 8 || ldx % 8 || ldq % 8 || ldx < K || ldq < K)
    return fail("dfh_quant_act_i8: K, ldx, ldq must be multiples of 8 with ld >= K (M=%d K=%d)", M, K);
  hipError_t e = quant_rows_bf16(reinterpret_cast<const uint16_t*>(x), ldx, reinterpret_cast<int8_t*>(q), ldq,
                                 reinterpret_cast<float*>(scale), M, K, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail("dfh_quant_act_i8: %s", hipGetErrorString(e));
  return 0;
}

int dfh_quant_weight_i8(const void* w, void* q, void* scale, int N, int K, void* stream) {
  if (!w || !q || !scale) return fail("dfh_quant_weight_i8: NULL pointer");
  if (N < 0 || K <= 0) return fail("dfh_quant_weight_i8: bad shape N=%d K=%d", N, K);
  hipError_t e = quant_weight_f32(reinterpret_cast<const uint16_t*>(w), reinterpret_cast<int8_t*>(q),
                                  reinterpret_cast<float*>(scale), N, K, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail("dfh_quant_weight_i8: %s", hipGetErrorString(e));
  return 0;
}

int dfh_gemm_w8a8(const void* xq, long ldx, const void* wq, long ldw, void* out, long ldo, const void* sx,
                  const void* sw, const void* bias, int M, int N, int K, int out_int32, int tile, void* stream) {
  return dfh_gemm_w8a8_ws(xq, ldx, wq, ldw, out, ldo, sx, sw, bias, M, N, K, out_int32, tile, nullptr, 0, stream);
}

int dfh_gemm_w8a8_ws(const void* xq, long ldx, const void* wq, long ldw, void* out, long ldo, const void* sx,
                     const void* sw, const void* bias, int M, int N, int K, int out_int32, int tile, void* ws,
                     long ws_bytes, void* stream) {
  if (!xq || !wq || !out) return fail("dfh_gemm_w8a8: NULL pointer");
  if (!out_int32 && (!sx || !sw)) return fail("dfh_gemm_w8a8: dequantised output needs both scales");
  if (K % 64 || ldx % 16 || ldw % 16 || ldx < K || ldw < K || ldo < N || ldo % 4)
    return fail("dfh_gemm_w8a8: K must be a multiple of 64, ldx/ldw multiples of 16 (M=%d N=%d K=%d)", M, N, K);
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = reinterpret_cast<const uint16_t*>(xq); a.lda = ldx;
  a.B = reinterpret_cast<const uint16_t*>(wq); a.ldb = ldw;
  a.C = reinterpret_cast<uint16_t*>(out); a.Ci = reinterpret_cast<int*>(out); a.ldc = ldo;
  a.sx = reinterpret_cast<const float*>(sx); a.sw = reinterpret_cast<const float*>(sw);
  a.bias = reinterpret_cast<const uint16_t*>(bias);
  a.M = M; a.N = N; a.K = K;
  a.ws = reinterpret_cast<float*>(ws); a.ws_elems = ws ? ws_bytes / 4 : 0;
  hipError_t e = gemm_i8(a, out_int32 ? EPI_I32 : EPI_DQ, reinterpret_cast<hipStream_t>(stream), tile);
  if (e != hipSuccess)
    return fail("dfh_gemm_w8a8(M=%d N=%d K=%d tile=%d): %s", M, N, K, tile, hipGetErrorString(e));
  return 0;
}

}  // extern "C"

// ===========================================================================
// Prefix K/V cache of a MeanFlow solve (the per-(timestep, layer) cache of
// nanovllm_dots/models/dots/cached_fm.py:82-197 for the MeanFlow DiT).
// History rows attend causally among themselves, so at a fixed timestep their
// K/V never depend on the latent: they are computed once per timestep (all
// timesteps in one batched prefix pass) and kept; each solver step then runs
// only the 1 + P active rows, which see the cached prefix and each other.
// Slab layout per layer: q|k rows [S*n*cap, 2H] and V^T [H, S*n*cap + 256];
// region (k, i) = rows / columns [(k*n + i) * cap, +cap) holds stream i's prefix
// at timestep k, followed by scratch slots for the step's active rows.
struct DfhKVCache {
  DfhHandle* h = nullptr;
  int n = 0, S = 0, cap = 0;  // cap: region stride (the capacity rounded up to 64 keys)
  int capacity = 0;           // rows a stream may hold, prefix + active block
  long rows_total = 0, ld_vt = 0;
  std::vector<DevBuf> qk, vt;
  DevBuf lens, counts, offs, seqs, c_rows, row_req, row_pos, vt_col, patch_rows, lh_rows, part, part_cnt, z;
  long table_rows = 0;
  std::vector<int> lens_host;
  // extend's uploads (counts, prefix sums: 2n + 2 ints) go through a ring of
  // pinned slots; a slot is rewritten once the event recorded after its copies
  // has completed, kPinnedSlots calls later, so the host does not wait on the stream
  static constexpr int kPinnedSlots = 8;
  int* pinned = nullptr;
  hipEvent_t pinned_ev[kPinnedSlots] = {};
  bool pinned_used[kPinnedSlots] = {};
  int pinned_next = 0;
};

namespace {

int cache_tables(DfhKVCache* c, long rows, hipStream_t s) {
  if (rows <= c->table_rows) return 0;
  DFH_CHECK(hipStreamSynchronize(s));
  DFH_CHECK(dev_alloc(c->c_rows, rows * 4));
  DFH_CHECK(dev_alloc(c->row_req, rows * 4));
  DFH_CHECK(dev_alloc(c->row_pos, rows * 4));
  DFH_CHECK(dev_alloc(c->vt_col, rows * 4));
  c->table_rows = rows;
  return 0;
}

Pass cache_pass(DfhKVCache* c) {
  DfhHandle* h = c->h;
  Pass p;
  for (int l = 0; l < h->cfg.n_blocks; ++l) {
    p.qk.push_back(P<uint16_t>(c->qk[l]));
    p.vt.push_back(P<uint16_t>(c->vt[l]));
  }
  p.ldqk = qk_stride(h->cfg);
  p.ld_vt = c->ld_vt;
  return p;
}

// Append counts[i] rows (FM sequence space, before input_layer) to each
// stream's prefix at every timestep. rows: device bf16, stream i's rows start at
// rows + i * stride (elements), consecutive rows H apart. counts/offs: device.
int cache_extend_dev(DfhKVCache* c, const uint16_t* rows, long stride, int m_max, int Mtot, int max_count,
                     const uint16_t* g, const TimeVals& tv, const TimeVals& dtv, hipStream_t s) {
  DfhHandle* h = c->h;
  const DfhConfig& cf = h->cfg;
  const long total = (long)c->S * Mtot;
  if (total == 0) return 0;
  if (total * (cf.ffn > qk_stride(cf) ? cf.ffn : qk_stride(cf)) >= (1L << 31))
    return fail("kv cache extend: %ld rows too many for one pass (32-bit element offsets)", total);
  if (reserve(h, c->n, c->cap, c->S, s)) return 1;  // RoPE positions up to cap
  if (reserve_rows(h, total, s)) return 1;
  if (cache_tables(c, total, s)) return 1;
  // positions up to cap
  DFH_CHECK(rope_table(P<float>(h->consts), cf.head_dim / 2, c->cap, P<float>(c->h->rope_cos),
                       P<float>(c->h->rope_sin), s));
  if (build_modulation(h, c->S, c->n, false, nullptr, nullptr, tv, dtv, true, g, s)) return 1;
  DFH_CHECK(prefix_tables(rows, stride, m_max, cf.hidden, P<int>(c->counts), P<int>(c->lens), P<int>(c->offs),
                          c->n, c->S, c->cap, P<uint16_t>(h->seq), P<int>(c->row_req), P<int>(c->row_pos),
                          P<int>(c->c_rows), P<int>(c->vt_col), P<AttnSeq>(c->seqs), s));
  Pass p = cache_pass(c);
  p.Mup = (int)total;
  p.row_req = P<int>(c->row_req);
  p.row_pos = P<int>(c->row_pos);
  p.c_rows = P<int>(c->c_rows);
  p.vt_col = P<int>(c->vt_col);
  p.seqs = P<AttnSeq>(c->seqs);
  p.n_seq = c->S * c->n;
  p.max_q = max_count;
  p.kv_only_last = true;
  if (run_blocks(h, p, s)) return 1;
  DFH_CHECK(cache_advance(P<int>(c->lens), P<int>(c->counts), c->n, s));
  return 0;
}

// NFE-step solve of the active rows against the cache.
int cache_solve(DfhKVCache* c, const uint16_t* last_hidden, const int* lh_src_rows, const uint16_t* g,
                const uint16_t* noise, uint16_t* out, const TimeVals& tv, const TimeVals& dtv, int max_len,
                hipStream_t s) {
  DfhHandle* h = c->h;
  const DfhConfig& cf = h->cfg;
  const int n = c->n, S = c->S, Pp = cf.patch, R = 1 + Pp, H = cf.hidden, ld = cf.latent_dim;
  const int rows = n * R;
  if (reserve(h, n, c->cap, S, s)) return 1;
  if (reserve_rows(h, rows, s)) return 1;
  if (cache_tables(c, (long)S * rows, s)) return 1;
  DFH_CHECK(rope_table(P<float>(h->consts), cf.head_dim / 2, c->cap, P<float>(h->rope_cos),
                       P<float>(h->rope_sin), s));
  if (build_modulation(h, S, n, false, nullptr, nullptr, tv, dtv, true, g, s)) return 1;
  DFH_CHECK(active_tables(P<int>(c->lens), n, S, Pp, c->cap, P<int>(c->row_req), P<int>(c->row_pos),
                          P<int>(c->c_rows), P<int>(c->vt_col), P<AttnSeq>(c->seqs), P<int>(c->patch_rows),
                          P<int>(c->lh_rows), s));
  // the last hidden rows of the active block (they stay put across steps)
  DFH_CHECK(gather_rows(last_hidden, lh_src_rows, P<int>(c->lh_rows), n, H, P<uint16_t>(h->seq), s));
  DFH_CHECK(hipMemcpyAsync(c->z.p, noise, (size_t)n * Pp * ld * 2, hipMemcpyDeviceToDevice, s));
  const int NP = n * Pp;
  for (int st = 0; st < S; ++st) {
    DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(c->z), ld, h->coord_w, h->coord_b,
                                            P<uint16_t>(h->zp), H, NP, nullptr, H, ld), EPI_BIAS, s));
    DFH_CHECK(scatter_rows(P<uint16_t>(h->zp), P<int>(c->patch_rows), NP, H, P<uint16_t>(h->seq), s));
    Pass p = cache_pass(c);
    p.Mup = rows;
    p.row_req = P<int>(c->row_req) + (long)st * rows;
    p.row_pos = P<int>(c->row_pos) + (long)st * rows;
    p.c_rows = P<int>(c->c_rows) + (long)st * rows;
    p.vt_col = P<int>(c->vt_col) + (long)st * rows;
    p.seqs = P<AttnSeq>(c->seqs) + (long)st * n;
    p.n_seq = n;
    p.max_kv = max_len + R;
    p.decode = true;
    p.part = P<float>(c->part);
    p.part_cnt = P<unsigned>(c->part_cnt);
    if (run_blocks(h, p, s)) return 1;
    const uint16_t* mf = P<uint16_t>(h->mod) + (long)cf.n_blocks * 6 * H;
    prof_arm(h, PC_LN);
    DFH_CHECK(ln_modulate(P<uint16_t>(h->x), H, P<uint16_t>(h->fin), H, mf, mf + H, h->ld_mod,
                          p.row_req, P<int>(c->patch_rows), NP, nullptr, H, cf.ln_eps, s));
    DFH_CHECK(gemm(h, PC_OTHER, linear_args(P<uint16_t>(h->fin), H, h->fin_w, h->fin_b,
                                            P<uint16_t>(h->vel), ld, NP, nullptr, ld, H), EPI_BIAS, s));
    DFH_CHECK(z_update(P<uint16_t>(c->z), P<uint16_t>(h->vel), dtv.v[st], (long)NP * ld, s));
  }
  DFH_CHECK(hipMemcpyAsync(out, c->z.p, (size_t)NP * ld * 2, hipMemcpyDeviceToDevice, s));
  return 0;
}

int cache_alloc(DfhHandle* h, int n, int cap, int S, DfhKVCache** out) {
  const DfhConfig& cf = h->cfg;
  DfhKVCache* c = new DfhKVCache();
  c->h = h; c->n = n; c->S = S; c->cap = cap;
  c->rows_total = (long)S * n * cap;
  c->ld_vt = c->rows_total + 256;
  c->qk.resize(cf.n_blocks);
  c->vt.resize(cf.n_blocks);
  auto bail = [&](hipError_t e) {
    for (auto& b : c->qk) if (b.p) (void)hipFree(b.p);
    for (auto& b : c->vt) if (b.p) (void)hipFree(b.p);
    DevBuf* bufs[] = {&c->lens, &c->counts, &c->offs, &c->seqs, &c->patch_rows, &c->lh_rows, &c->part,
                      &c->part_cnt, &c->z};
    for (DevBuf* b : bufs) if (b->p) (void)hipFree(b->p);
    if (c->pinned) (void)hipHostFree(c->pinned);
    for (hipEvent_t ev : c->pinned_ev) if (ev) (void)hipEventDestroy(ev);
    delete c;
    return fail("kv cache allocation: %s", hipGetErrorString(e));
  };
  for (int l = 0; l < cf.n_blocks; ++l) {
    hipError_t e = dev_alloc(c->qk[l], (size_t)c->rows_total * qk_stride(cf) * 2);
    if (e == hipSuccess) e = dev_alloc(c->vt[l], (size_t)cf.hidden * c->ld_vt * 2);
    if (e != hipSuccess) return bail(e);
  }
  DevBuf* small[] = {&c->lens, &c->counts, &c->offs};
  for (DevBuf* b : small) {
    hipError_t e = dev_alloc(*b, (size_t)(n + 1) * 4);
    if (e != hipSuccess) return bail(e);
  }
  const int n_chunks = (cap + 255) / 256;
  hipError_t e = dev_alloc(c->seqs, (size_t)S * n * sizeof(AttnSeq));
  if (e == hipSuccess) e = dev_alloc(c->patch_rows, (size_t)n * cf.patch * 4);
  if (e == hipSuccess) e = dev_alloc(c->lh_rows, (size_t)n * 4);
  if (e == hipSuccess) e = dev_alloc(c->part, (size_t)n * cf.heads * n_chunks * 32 * 66 * 4);
  if (e == hipSuccess) e = dev_alloc(c->part_cnt, (size_t)n * cf.heads * 4);  // zero-filled
  if (e == hipSuccess) e = dev_alloc(c->z, (size_t)n * cf.patch * cf.latent_dim * 2);
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&c->pinned), (size_t)DfhKVCache::kPinnedSlots * (2 * n + 2) * sizeof(int));
  for (int k = 0; k < DfhKVCache::kPinnedSlots && e == hipSuccess; ++k)
    e = hipEventCreateWithFlags(&c->pinned_ev[k], hipEventDisableTiming);
  if (e != hipSuccess) return bail(e);
  c->lens_host.assign(n, 0);
  *out = c;
  return 0;
}

}  // namespace

extern "C" {

int dfh_kvcache_create(DfhHandle* h, int n_streams, int capacity, int num_steps, DfhKVCache** out) {
  if (!h || !out) return fail("null argument");
  if (!h->weights_set) return fail("dfh_kvcache_create: weights not set");
  if (n_streams <= 0 || n_streams > 1024 || num_steps <= 0 || num_steps > kMaxTimeVals)
    return fail("dfh_kvcache_create: bad n_streams=%d num_steps=%d", n_streams, num_steps);
  if (capacity < h->cfg.patch + 2) return fail("dfh_kvcache_create: capacity %d too small", capacity);
  // the decode attention and its chunk merge hold the 1 + P active queries of a
  // stream in one 32-row MFMA block
  if (h->cfg.patch + 1 > 32)
    return fail("dfh_kvcache_create: latent patch %d too large (1 + patch active rows must be <= 32)",
                h->cfg.patch);
  // region starts at multiples of 64 keys: a 64-key V^T row segment is one 128-B line
  const int cap = (capacity + 63) & ~63;
  if ((long)num_steps * n_streams * cap * qk_stride(h->cfg) >= (1L << 31))
    return fail("dfh_kvcache_create: cache too large for 32-bit offsets");
  if (cache_alloc(h, n_streams, cap, num_steps, out)) return 1;
  (*out)->capacity = capacity;
  return 0;
}

int dfh_kvcache_destroy(DfhKVCache* c) {
  if (!c) return 0;
  (void)hipDeviceSynchronize();
  for (auto& b : c->qk) if (b.p) (void)hipFree(b.p);
  for (auto& b : c->vt) if (b.p) (void)hipFree(b.p);
  DevBuf* bufs[] = {&c->lens, &c->counts, &c->offs, &c->seqs, &c->c_rows, &c->row_req, &c->row_pos,
                    &c->vt_col, &c->patch_rows, &c->lh_rows, &c->part, &c->part_cnt, &c->z};
  for (DevBuf* b : bufs) if (b->p) (void)hipFree(b->p);
  if (c->pinned) (void)hipHostFree(c->pinned);
  for (hipEvent_t ev : c->pinned_ev) if (ev) (void)hipEventDestroy(ev);
  delete c;
  return 0;
}

int dfh_kvcache_reset(DfhKVCache* c, void* stream) {
  if (!c) return fail("null cache");
  DFH_CHECK(hipMemsetAsync(c->lens.p, 0, (size_t)c->n * 4, reinterpret_cast<hipStream_t>(stream)));
  c->lens_host.assign(c->n, 0);
  return 0;
}

int dfh_kvcache_lengths(DfhKVCache* c, int* lens) {
  if (!c || !lens) return fail("null argument");
  for (int i = 0; i < c->n; ++i) lens[i] = c->lens_host[i];
  return 0;
}

int dfh_kvcache_extend(DfhKVCache* c, const void* rows, int m_max, const int* counts, const void* g_cond,
                       const float* t_grid, const float* dt_grid, void* stream) {
  if (!c || !rows || !counts || !t_grid || !dt_grid) return fail("dfh_kvcache_extend: NULL argument");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int R = 1 + c->h->cfg.patch;
  int Mtot = 0, max_count = 0;
  for (int i = 0; i < c->n; ++i) {
    if (counts[i] < 0 || counts[i] > m_max) return fail("dfh_kvcache_extend: counts[%d]=%d", i, counts[i]);
    if (c->lens_host[i] + counts[i] + R > c->capacity)
      return fail("dfh_kvcache_extend: stream %d would hold %d rows (+%d active) > capacity %d", i,
                  c->lens_host[i] + counts[i], R, c->capacity);
    Mtot += counts[i];
    max_count = counts[i] > max_count ? counts[i] : max_count;
  }
  if (Mtot == 0) return 0;
  // stage counts and their exclusive prefix sums in the next pinned slot
  const int slot = c->pinned_next;
  c->pinned_next = (slot + 1) % DfhKVCache::kPinnedSlots;
  if (c->pinned_used[slot]) DFH_CHECK(hipEventSynchronize(c->pinned_ev[slot]));
  int* pin = c->pinned + (size_t)slot * (2 * c->n + 2);
  int acc = 0;
  for (int i = 0; i < c->n; ++i) { pin[i] = counts[i]; pin[c->n + 1 + i] = acc; acc += counts[i]; }
  pin[2 * c->n + 1] = acc;
  DFH_CHECK(hipMemcpyAsync(c->counts.p, pin, (size_t)c->n * 4, hipMemcpyHostToDevice, s));
  DFH_CHECK(hipMemcpyAsync(c->offs.p, pin + c->n + 1, (size_t)(c->n + 1) * 4, hipMemcpyHostToDevice, s));
  DFH_CHECK(hipEventRecord(c->pinned_ev[slot], s));
  c->pinned_used[slot] = true;
  TimeVals tv{}, dtv{};
  for (int k = 0; k < c->S; ++k) { tv.v[k] = t_grid[k]; dtv.v[k] = dt_grid[k]; }
  const int H = c->h->cfg.hidden;
  if (cache_extend_dev(c, reinterpret_cast<const uint16_t*>(rows), (long)m_max * H, m_max, Mtot, max_count,
                       reinterpret_cast<const uint16_t*>(g_cond), tv, dtv, s))
    return 1;
  for (int i = 0; i < c->n; ++i) c->lens_host[i] += counts[i];
  return 0;
}

int dfh_kvcache_solve(DfhKVCache* c, const void* last_hidden, const void* g_cond, const void* noise, void* out,
                      const float* t_grid, const float* dt_grid, void* stream) {
  if (!c || !last_hidden || !noise || !out || !t_grid || !dt_grid) return fail("dfh_kvcache_solve: NULL argument");
  const int R = 1 + c->h->cfg.patch;
  int max_len = 0;
  for (int i = 0; i < c->n; ++i) {
    if (c->lens_host[i] + R > c->capacity) return fail("dfh_kvcache_solve: stream %d prefix too long", i);
    max_len = c->lens_host[i] > max_len ? c->lens_host[i] : max_len;
  }
  TimeVals tv{}, dtv{};
  for (int k = 0; k < c->S; ++k) { tv.v[k] = t_grid[k]; dtv.v[k] = dt_grid[k]; }
  return cache_solve(c, reinterpret_cast<const uint16_t*>(last_hidden), nullptr,
                     reinterpret_cast<const uint16_t*>(g_cond), reinterpret_cast<const uint16_t*>(noise),
                     reinterpret_cast<uint16_t*>(out), tv, dtv, max_len, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"

// ----------------------------------------------------------------------------
// Patch encoder decode (FlashPatchEncoder.decode_patch, flash_patch_encoder.py
// :103-139). Per call, stream-ordered: per-call tables (K/V slots, key counts,
// query offsets) from the rows' lengths; causal downsample of each request's
// patch (conv tail in, new tail out) and in_proj; per layer LayerNorm, fused
// q|k|v GEMM, K / V rows appended to the cache, paged attention with one page
// per cache row (block_table = rows), o_proj with an in-place residual add,
// LayerNorm, fc1 + SiLU, fc2 with an in-place residual add; the rows' lengths
// advance; out_proj over each request's patch / 2 tokens side by side.
// ----------------------------------------------------------------------------
struct DfhPatchEnc {
  DfhPatchEncConfig cfg;
  int ods = 0, cap = 0;
  DevBuf arena;  // packed weights
  const uint16_t *ds_w, *ds_b, *in_w, *in_b, *out_w, *out_b;
  std::vector<const uint16_t*> ln1_w, ln1_b, qkv_w, o_w, o_b, ln2_w, ln2_b, fc1_w, fc1_b, fc2_w, fc2_b;
  DevBuf kc, vc;                 // [n_layers][max_batch * cap][hidden]
  DevBuf len, tail, err;         // per row: length, conv tail [latent_dim]; overflow flag
  DevBuf x, hb, qkv, attn, ff, conv, slots, seqk, cuq, zeros, ones, paws;
  DevBuf rows_ok;                // the call's rows, out-of-range entries replaced by row 0
};

namespace {
int pe_gemm(const uint16_t* A, long lda, const uint16_t* B, const uint16_t* bias, uint16_t* C, long ldc, int M,
            int N, int K, int epi, const DfhPatchEnc* h, hipStream_t s) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.A = A; a.lda = lda; a.B = B; a.ldb = K; a.C = C; a.ldc = ldc; a.bias = bias;
  a.M = M; a.N = N; a.K = K;
  if (epi == EPI_GATE_RES) {  // x += bf16(acc + bias): unit gate for every row
    a.gate = P<const uint16_t>(const_cast<DevBuf&>(h->ones)); a.ld_gate = 0;
    a.row_req = P<const int>(const_cast<DevBuf&>(h->zeros));
  }
  hipError_t e = gemm_bf16(a, epi, s, -1);
  if (e != hipSuccess) return fail("patch encoder GEMM (M=%d N=%d K=%d epi=%d): %s", M, N, K, epi, hipGetErrorString(e));
  return 0;
}
}  // namespace

extern "C" {

int dfh_patchenc_create(const DfhPatchEncConfig* cfg, const DfhPatchEncWeights* w, DfhPatchEnc** out) {
  if (!cfg || !w || !out || !w->layers) return fail("dfh_patchenc_create: NULL argument");
  const DfhPatchEncConfig& c = *cfg;
  if (c.hidden <= 0 || c.heads <= 0 || c.hidden % c.heads || c.hidden % 256)
    return fail("dfh_patchenc_create: hidden %d must be a positive multiple of 256 and of heads %d", c.hidden,
                c.heads);
  const int hd = c.hidden / c.heads;
  if (hd != 64 && hd != 128) return fail("dfh_patchenc_create: head_dim %d not supported (64 or 128)", hd);
  if (c.latent_dim <= 0 || c.latent_dim % 32 || c.patch <= 0 || c.patch % 2 || c.out_dim <= 0 || c.out_dim % 64 ||
      c.ffn <= 0 || c.ffn % 64 || c.n_layers <= 0 || c.max_batch <= 0 || c.capacity <= 0)
    return fail("dfh_patchenc_create: bad shape (latent_dim %d, patch %d, ffn %d, out_dim %d, layers %d, rows %d, "
                "capacity %d)", c.latent_dim, c.patch, c.ffn, c.out_dim, c.n_layers, c.max_batch, c.capacity);
  if ((long)(c.patch + 1) * c.latent_dim * 4 > 64 * 1024) return fail("dfh_patchenc_create: patch too large");
  auto* h = new DfhPatchEnc();
  h->cfg = c;
  h->ods = c.patch / 2;
  h->cap = (c.capacity + 255) / 256 * 256;
  const long H = c.hidden, F = c.ffn, L = c.latent_dim, rows_max = (long)c.max_batch * h->ods;
  auto fail_free = [&](int rc) {
    dfh_patchenc_destroy(h);
    return rc;
  };
  // weight arena: 256-B aligned pieces
  std::vector<std::pair<const void*, long>> pieces;  // (source, elements)
  auto add = [&](const void* src, long n) { pieces.push_back({src, n}); };
  add(w->ds_w, L * L * 2); add(w->ds_b, L); add(w->in_w, H * L); add(w->in_b, H);
  add(w->out_w, (long)c.out_dim * H * h->ods); add(w->out_b, c.out_dim);
  for (int l = 0; l < c.n_layers; ++l) {
    const DfhPatchEncLayerWeights& lw = w->layers[l];
    add(lw.attn_norm_w, H); add(lw.attn_norm_b, H);
    add(lw.q_w, H * H); add(lw.k_w, H * H); add(lw.v_w, H * H);  // consecutive: the fused [3H, H] q|k|v
    add(lw.o_w, H * H); add(lw.o_b, H);
    add(lw.ffn_norm_w, H); add(lw.ffn_norm_b, H);
    add(lw.fc1_w, F * H); add(lw.fc1_b, F); add(lw.fc2_w, H * F); add(lw.fc2_b, H);
  }
  std::vector<long> offs;
  long total = 0;
  for (auto& p : pieces) {
    if (!p.first) return fail_free(fail("dfh_patchenc_create: a weight pointer is NULL"));
    offs.push_back(total);
    total += p.second * 2;
    total = (total + 255) / 256 * 256;
  }
  // q, k, v of a layer must be contiguous for the fused GEMM: their sizes (H*H*2 bytes) are multiples of 256
  if (dev_alloc(h->arena, total) != hipSuccess) return fail_free(fail("dfh_patchenc_create: weight allocation"));
  for (size_t i = 0; i < pieces.size(); ++i)
    if (hipMemcpy(reinterpret_cast<char*>(h->arena.p) + offs[i], pieces[i].first, pieces[i].second * 2,
                  hipMemcpyDeviceToDevice) != hipSuccess)
      return fail_free(fail("dfh_patchenc_create: weight copy %zu failed", i));
  auto at = [&](size_t i) { return reinterpret_cast<const uint16_t*>(reinterpret_cast<char*>(h->arena.p) + offs[i]); };
  size_t k = 0;
  h->ds_w = at(k++); h->ds_b = at(k++); h->in_w = at(k++); h->in_b = at(k++); h->out_w = at(k++); h->out_b = at(k++);
  for (int l = 0; l < c.n_layers; ++l) {
    h->ln1_w.push_back(at(k++)); h->ln1_b.push_back(at(k++));
    h->qkv_w.push_back(at(k)); k += 3;
    h->o_w.push_back(at(k++)); h->o_b.push_back(at(k++));
    h->ln2_w.push_back(at(k++)); h->ln2_b.push_back(at(k++));
    h->fc1_w.push_back(at(k++)); h->fc1_b.push_back(at(k++)); h->fc2_w.push_back(at(k++)); h->fc2_b.push_back(at(k++));
  }
  const size_t cache = (size_t)c.n_layers * c.max_batch * h->cap * H * 2;
  // a call with fewer requests may split rows into more chunks: the largest need over every batch size
  long pa_ws = 0;
  for (int nb = 1; nb <= c.max_batch; ++nb) {
    const long need = dfh::paged_attention_ws_bytes(nb, c.heads, 1, h->ods, h->cap, hd, (long)nb * h->ods);
    pa_ws = need > pa_ws ? need : pa_ws;
  }
  std::vector<uint16_t> ones(H, 0x3f80);  // bf16 1.0
  if (dev_alloc(h->kc, cache) || dev_alloc(h->vc, cache) || dev_alloc(h->len, (size_t)c.max_batch * 4) ||
      dev_alloc(h->tail, (size_t)c.max_batch * L * 2) || dev_alloc(h->err, 256) ||
      dev_alloc(h->x, rows_max * H * 2) || dev_alloc(h->hb, rows_max * H * 2) ||
      dev_alloc(h->qkv, rows_max * 3 * H * 2) || dev_alloc(h->attn, rows_max * H * 2) ||
      dev_alloc(h->ff, rows_max * F * 2) || dev_alloc(h->conv, rows_max * L * 2) ||
      dev_alloc(h->slots, rows_max * 4) || dev_alloc(h->seqk, (size_t)c.max_batch * 4) ||
      dev_alloc(h->cuq, (size_t)(c.max_batch + 1) * 4) || dev_alloc(h->zeros, rows_max * 4) ||
      dev_alloc(h->ones, H * 2) || dev_alloc(h->paws, pa_ws > 0 ? pa_ws : 256) ||
      dev_alloc(h->rows_ok, (size_t)c.max_batch * 4) ||
      hipMemcpy(h->ones.p, ones.data(), H * 2, hipMemcpyHostToDevice))
    return fail_free(fail("dfh_patchenc_create: allocation of %.1f MiB of caches failed", 2.0 * cache / (1 << 20)));
  *out = h;
  return 0;
}

int dfh_patchenc_destroy(DfhPatchEnc* h) {
  if (!h) return 0;
  (void)hipDeviceSynchronize();
  for (DevBuf* b : {&h->arena, &h->kc, &h->vc, &h->len, &h->tail, &h->err, &h->x, &h->hb, &h->qkv, &h->attn, &h->ff,
                    &h->conv, &h->slots, &h->seqk, &h->cuq, &h->zeros, &h->ones, &h->paws, &h->rows_ok})
    if (b->p) (void)hipFree(b->p);
  delete h;
  return 0;
}

int dfh_patchenc_reset_rows(DfhPatchEnc* h, const int* rows, int n, void* stream) {
  if (!h) return fail("dfh_patchenc_reset_rows: NULL handle");
  if (n < 0 || n > h->cfg.max_batch || (n > 0 && !rows))
    return fail("dfh_patchenc_reset_rows: %d rows (the handle has %d)", n, h->cfg.max_batch);
  DFH_CHECK(pe_reset(rows, n, h->cfg.max_batch, P<int>(h->len), P<uint16_t>(h->tail), h->cfg.latent_dim,
                     reinterpret_cast<hipStream_t>(stream)));
  return 0;
}

int dfh_patchenc_decode(DfhPatchEnc* h, const void* patches, long patch_stride, const int* rows, int n, void* out,
                        void* stream) {
  if (!h) return fail("dfh_patchenc_decode: NULL handle");
  if (n == 0) return 0;
  if (n < 0 || n > h->cfg.max_batch)
    return fail("dfh_patchenc_decode: %d requests (the handle has %d rows)", n, h->cfg.max_batch);
  if (!patches || !rows || !out) return fail("dfh_patchenc_decode: NULL pointer");
  const DfhPatchEncConfig& c = h->cfg;
  if (patch_stride < (long)c.patch * c.latent_dim) return fail("dfh_patchenc_decode: patch_stride too small");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int H = c.hidden, F = c.ffn, L = c.latent_dim, ods = h->ods, M = n * ods;
  const long lstride = (long)c.max_batch * h->cap * H;  // one layer's cache, elements
  DFH_CHECK(pe_plan(rows, P<int>(h->len), n, ods, h->cap, c.max_batch, P<int>(h->rows_ok), P<int>(h->slots),
                    P<int>(h->seqk), P<int>(h->cuq), P<int>(h->err), s));
  rows = P<const int>(h->rows_ok);  // the caller's rows, range-checked
  DFH_CHECK(pe_downsample(reinterpret_cast<const uint16_t*>(patches), patch_stride, h->ds_w, h->ds_b, rows,
                          P<uint16_t>(h->tail), P<uint16_t>(h->conv), n, c.patch, L, s));
  uint16_t* x = P<uint16_t>(h->x);
  uint16_t* hb = P<uint16_t>(h->hb);
  uint16_t* qkv = P<uint16_t>(h->qkv);
  uint16_t* attn = P<uint16_t>(h->attn);
  uint16_t* ff = P<uint16_t>(h->ff);
  if (pe_gemm(P<uint16_t>(h->conv), L, h->in_w, h->in_b, x, H, M, H, L, EPI_BIAS, h, s)) return 1;
  for (int l = 0; l < c.n_layers; ++l) {
    uint16_t* kc = P<uint16_t>(h->kc) + l * lstride;
    uint16_t* vc = P<uint16_t>(h->vc) + l * lstride;
    DFH_CHECK(ln_affine(x, hb, h->ln1_w[l], h->ln1_b[l], M, H, c.ln_eps, s));
    if (pe_gemm(hb, H, h->qkv_w[l], nullptr, qkv, 3 * H, M, 3 * H, H, EPI_BIAS, h, s)) return 1;
    DFH_CHECK(store_kvcache(qkv + H, 3 * H, qkv + 2 * H, 3 * H, kc, vc, P<int>(h->slots), M, H, s));
    PagedAttnArgs pa{};
    pa.batch = n; pa.heads = c.heads; pa.kv_heads = c.heads; pa.head_dim = H / c.heads;
    pa.max_q = ods; pa.max_k = h->cap; pa.total_q = M;
    pa.q = qkv; pa.q_stride = 3 * H; pa.cu_q = P<int>(h->cuq);
    pa.k = kc; pa.v = vc; pa.kv_stride = H; pa.cu_k = nullptr; pa.seqlens_k = P<int>(h->seqk);
    pa.block_table = rows; pa.bt_stride = 1; pa.block_size = h->cap;
    pa.out = attn; pa.out_stride = H; pa.scale = 1.0f / sqrtf((float)(H / c.heads)); pa.causal = 1;
    pa.ws = h->paws.p;
    if (dfh::paged_attention_ws_bytes(n, c.heads, 1, ods, h->cap, H / c.heads, M) > (long)h->paws.bytes)
      return fail("dfh_patchenc_decode: attention workspace too small for %d requests", n);
    DFH_CHECK(paged_attention(pa, s));
    if (pe_gemm(attn, H, h->o_w[l], h->o_b[l], x, H, M, H, H, EPI_GATE_RES, h, s)) return 1;
    DFH_CHECK(ln_affine(x, hb, h->ln2_w[l], h->ln2_b[l], M, H, c.ln_eps, s));
    if (pe_gemm(hb, H, h->fc1_w[l], h->fc1_b[l], ff, F, M, F, H, EPI_SILU, h, s)) return 1;
    if (pe_gemm(ff, F, h->fc2_w[l], h->fc2_b[l], x, H, M, H, F, EPI_GATE_RES, h, s)) return 1;
  }
  DFH_CHECK(pe_advance(rows, P<int>(h->len), n, ods, h->cap, s));
  // request i's ods tokens are consecutive rows: one [n, ods * H] row each
  if (pe_gemm(x, (long)ods * H, h->out_w, h->out_b, reinterpret_cast<uint16_t*>(out), c.out_dim, n, c.out_dim,
              ods * H, EPI_BIAS, h, s))
    return 1;
  return 0;
}

int dfh_patchenc_lengths(DfhPatchEnc* h, int* lengths, int* overflow) {
  if (!h) return fail("dfh_patchenc_lengths: NULL handle");
  DFH_CHECK(hipDeviceSynchronize());
  if (lengths) DFH_CHECK(hipMemcpy(lengths, h->len.p, (size_t)h->cfg.max_batch * 4, hipMemcpyDeviceToHost));
  int e = 0;
  DFH_CHECK(hipMemcpy(&e, h->err.p, 4, hipMemcpyDeviceToHost));
  if (overflow) *overflow = e;
  if (e) DFH_CHECK(hipMemset(h->err.p, 0, 4));
  return 0;
}

}  // extern "C"
