/* dots_fm.h — C ABI of the MI355X (gfx950) MeanFlow FM/DiT head.
 *
 * One shared library, libdotsfm.so. Plain C types only: device pointers are
 * `void*` (memory owned by the caller, e.g. torch tensors), host arrays are
 * plain pointers, streams are `void*` holding a hipStream_t (NULL = default
 * stream). Every function returns 0 on success or a nonzero status; the
 * message of the last failure on the calling thread is dfh_last_error().
 * No C++ exception crosses this boundary.
 *
 * Reference interfaces replaced (paths in the nanovllm_dots repository):
 *   dfh_meanflow_solve  <- GraphedMeanflow.__call__
 *                          nanovllm_dots/models/dots/graphed_meanflow.py:36-60, and
 *                          batched_meanflow nanovllm_dots/models/dots/batched_fm.py:82-126
 *   dfh_meanflow_solve_varlen
 *                       <- DotsBatchEngine._pack_fm_inputs + the solve call
 *                          nanovllm_dots/models/dots/engine.py:635-688, 713-724
 *   dfh_dit_forward     <- DiT.forward (the `vfp` callable)
 *                          nanovllm_dots/models/dots/native/dit.py:135-148
 *   dfh_set_weights     <- build_native_dit / load_component weight binding
 *                          nanovllm_dots/models/dots/native/loader.py:23-67
 *   dfh_gemm_bf16       <- nn.Linear (cuBLAS bf16 GEMM) as used by the DiT
 *                          nanovllm_dots/models/dots/native/layers.py:82-84, 152-161
 *   dfh_quant_act_i8, dfh_quant_weight_i8, dfh_gemm_w8a8
 *                       <- Int8DynamicLinear nanovllm_dots/models/dots/int8_dit.py:34-65
 *   dfh_store_kvcache   <- store_kvcache nanovllm_dots/layers/attention.py:10-47
 *   dfh_paged_attention <- flash_attn_varlen_func / flash_attn_with_kvcache as called
 *                          by Attention.forward nanovllm_dots/layers/attention.py:66-95
 *   dfh_kvcache_*       <- FMCache / extend_cache / active_forward
 *                          nanovllm_dots/models/dots/cached_fm.py:82-197 (CFG flow matching
 *                          there; restated for the MeanFlow DiT)
 */
#ifndef DOTS_FM_H
#define DOTS_FM_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct DfhHandle DfhHandle;
typedef struct DfhKVCache DfhKVCache;

/* DiT shape. Mirrors the checkpoint config's DiT block
 * (nanovllm_dots/models/dots/native/config.py:46-47, loader.py:52-67) and the core
 * scalars latent_dim / latent_patch_size (native/core.py:50-55).
 * Supported: head_dim == 64, hidden % 256 == 0, ffn % 256 == 0,
 * latent_dim % 64 == 0, freq_dim % 64 == 0. */
typedef struct DfhConfig {
  int hidden;
  int heads;
  int head_dim;
  int ffn;
  int n_blocks;
  int latent_dim;
  int patch;          /* latent rows per request (latent_patch_size) */
  int freq_dim;       /* timestep frequency embedding size (256) */
  int qkv_bias;       /* q/k/v projections carry a bias */
  int qk_norm;        /* 0 none, 1 LayerNorm(head_dim, affine), 2 RMSNorm(head_dim) */
  int rotary;         /* RoPE on q and k */
  int meanflow;       /* duration embedder present (MeanFlow DiT) */
  float ln_eps;       /* block / final LayerNorm eps (1e-5) */
  const float* rope_inv_freq;  /* host, head_dim/2 floats (RotaryEmbedding.inv_freq) */
  const float* temb_freqs;     /* host, freq_dim/2 floats (TimestepEmbedder freqs) */
} DfhConfig;

/* Device pointers to bf16 parameters in nn.Linear layout ([out, in] row-major),
 * named after the reference state dict. Optional tensors may be NULL. */
typedef struct DfhBlockWeights {
  const void *q_w, *q_b, *k_w, *k_b, *v_w, *v_b;       /* attn.{q,k,v}_proj */
  const void *q_norm_w, *q_norm_b, *k_norm_w, *k_norm_b; /* attn.{q,k}_norm */
  const void *o_w, *o_b;                                /* attn.o_proj */
  const void *fc1_w, *fc1_b, *fc2_w, *fc2_b;            /* ffn.fc1 / ffn.fc2 */
  const void *ada_w, *ada_b;                            /* adaLN_modulation.1 [6H, H] */
} DfhBlockWeights;

typedef struct DfhWeights {
  const void *input_w, *input_b;                 /* input_layer */
  const void *t_w0, *t_b0, *t_w2, *t_b2;         /* time_embedder.mlp.{0,2} */
  const void *d_w0, *d_b0, *d_w2, *d_b2;         /* duration_embedder.mlp.{0,2} */
  const void *final_ada_w, *final_ada_b;         /* output_layer.adaLN_modulation.1 [2H, H] */
  const void *final_w, *final_b;                 /* output_layer.linear [ld, H] */
  const void *coord_w, *coord_b;                 /* core.coordinate_proj [H, ld] */
  const DfhBlockWeights* blocks;                 /* host array of n_blocks */
} DfhWeights;

/* Whole MeanFlow solve over N padded requests (the input contract of
 * DotsBatchEngine._pack_fm_inputs, engine.py:635-688). The FM mask is implied
 * by pos_ids (history length c_i = pos_ids[i, T-P]) and is not read. */
typedef struct DfhSolveArgs {
  int n;                    /* requests */
  int total_len;            /* T = max history + patch */
  int num_steps;            /* NFE (<= 16) */
  const void* input_sequence;  /* bf16 [n, T, H], latent slot zero */
  const void* pos_ids;         /* f32  [n, T] */
  const void* g_cond;          /* bf16 [n, H] or NULL (zeros) */
  const void* noise;           /* bf16 [n, P, ld] */
  void* out;                   /* bf16 [n, P, ld] */
  const float* t_grid;         /* host [num_steps]: t_s */
  const float* dt_grid;        /* host [num_steps]: t_{s+1} - t_s */
} DfhSolveArgs;

/* Whole MeanFlow solve over N requests handed over as they sit in the engine
 * (varlen): request i's c_i = hist_len[i] history rows start at hist_rows[i],
 * row stride row_stride elements; no padded batch, no mask, no pos_ids.
 * This replaces the padding half of DotsBatchEngine._pack_fm_inputs
 * (engine.py:635-688: the per-request copies of fm_sequence[0, :L] into a
 * zero [n, max_len + P, H] batch, the [n, T, T] mask and pos_ids built by
 * _build_fm_attn_mask / _build_fm_pos_ids, native/model.py:57-87). The result
 * equals dfh_meanflow_solve on the padded batch of the same requests, bit for bit.
 * hist_rows: 16-B aligned bases; row_stride >= hidden, a multiple of 8.
 * A length outside [1, max_hist] or a misaligned base is reported by
 * dfh_input_status (bits 0 and 1), like a bad pos_ids in dfh_meanflow_solve;
 * such a request is solved with its first history row only (or zero rows). */
typedef struct DfhVarlenSolveArgs {
  int n;                    /* requests */
  int max_hist;             /* >= every c_i (sizes the workspace) */
  int num_steps;            /* NFE (<= 16) */
  const void* const* hist_rows;  /* device array [n] of device pointers to bf16 rows */
  const int* hist_len;           /* device int32 [n]: c_i */
  long row_stride;               /* elements between consecutive history rows */
  const void* g_cond;            /* bf16 [n, H] or NULL (zeros) */
  const void* noise;             /* bf16 [n, P, ld] */
  void* out;                     /* bf16 [n, P, ld] */
  const float* t_grid;           /* host [num_steps]: t_s */
  const float* dt_grid;          /* host [num_steps]: t_{s+1} - t_s */
} DfhVarlenSolveArgs;

/* One DiT forward (the vfp callable) on the padded layout. */
typedef struct DfhForwardArgs {
  int n;
  int total_len;
  const void* x;            /* bf16 [n, T, H] */
  const void* timesteps;    /* f32 [n] device */
  const void* duration;     /* f32 [n] device or NULL */
  const void* pos_ids;      /* f32 [n, T] */
  const void* g_cond;       /* bf16 [n, H] or NULL */
  void* out;                /* bf16 [n, T, ld]; padding rows are written as 0 */
} DfhForwardArgs;

const char* dfh_last_error(void);

int dfh_create(const DfhConfig* cfg, DfhHandle** out);
int dfh_destroy(DfhHandle* h);
/* Packs the weights into handle-owned device memory (fused QKV, one adaLN
 * matrix for all blocks). Synchronizes the stream. */
int dfh_set_weights(DfhHandle* h, const DfhWeights* w, void* stream);
/* Grows the workspace for up to n requests of padded length T and num_steps
 * solver steps (synchronizes the stream only when it grows). */
int dfh_reserve(DfhHandle* h, int n, int total_len, int num_steps, void* stream);
int dfh_meanflow_solve(DfhHandle* h, const DfhSolveArgs* a, void* stream);
int dfh_meanflow_solve_varlen(DfhHandle* h, const DfhVarlenSolveArgs* a, void* stream);
int dfh_dit_forward(DfhHandle* h, const DfhForwardArgs* a, void* stream);
/* Reads and clears the device-side input check of the last solve/forward
 * (bit 0: a pos_ids row does not describe a valid FM layout). Synchronizes. */
int dfh_input_status(DfhHandle* h, int* flags, void* stream);

/* Per-kernel-class timing with dispatch-packet events (bench instrumentation).
 * classes: 0 qkv gemm, 1 o_proj gemm, 2 fc1 gemm, 3 fc2 gemm, 4 attention,
 * 5 ln_modulate, 6 other, 7 the latent tail of the last block (see
 * dfh_set_latent_tail). */
int dfh_profile_enable(DfhHandle* h, int enable);
/* Which launches carry events while profiling is on: of the classes in mask
 * (bit c for class c; default all), launches 0, every, 2*every, ... of each
 * class, counted from this call (default every = 1: all). An evented launch
 * adds a few microseconds of dispatch before and after it, so a timed region
 * arms a sample of the class it measures. every < 1 is an error. */
int dfh_profile_classes(DfhHandle* h, unsigned mask, int every);
/* K-split of each GEMM's last, partial round of tiles (default on): leftover
 * tiles are cut along K over the idle workgroups; the workgroup that completes a
 * tile adds the partial sums. Off: every tile runs whole. No reference counterpart
 * (a scheduling choice of this library; results agree to float32 summation order). */
int dfh_set_ksplit(DfhHandle* h, int enable);
/* Latent tail of the MeanFlow solves (default on): the caller keeps only the P
 * latent rows of each DiT output (batched_fm.py:122-124), so the last block
 * runs LayerNorm + QKV over every row (the latent rows attend over all K/V) and
 * attention, O projection, LayerNorm and MLP over the latent rows alone; the
 * final layer reads them. Off: the last block runs over every row, as the
 * reference does. Both give the same latents up to float32 summation order.
 * No reference counterpart (an evaluation-order choice of this library). */
int dfh_set_latent_tail(DfhHandle* h, int enable);
int dfh_profile_read(DfhHandle* h, double* ms_per_class, long* launches_per_class, int n_classes);

/* Standalone bf16 GEMM: C[M,N] = A[M,K] B[N,K]^T + bias (bias may be NULL).
 * epilogue: 0 bf16 out, 1 GELU(tanh) bf16 out, 4 float32 out, 7 SiLU bf16 out. */
int dfh_gemm_bf16(const void* A, long lda, const void* B, long ldb, void* C, long ldc,
                  const void* bias, int M, int N, int K, int epilogue, int tile, void* stream);
/* W8A8 mode of dfh_meanflow_solve / dfh_meanflow_solve_varlen / dfh_dit_forward
 * and the cached solve <- quantize_dit_ + Int8DynamicLinear
 * (nanovllm_dots/models/dots/int8_dit.py:34-85). Every DiT linear with
 * min(in, out) >= 512 becomes W8A8: input_layer, the second linear of the time
 * and duration MLPs, every adaLN (stacked as in DfhWeights), q|k|v (fused), o,
 * fc1 and fc2. Per-output-channel int8 weights (float32 scales) come from the
 * caller (w, any entry NULL: quantised here from the handle's bf16 weights
 * exactly as Int8DynamicLinear does); the input rows of each linear are
 * quantised per token in bf16 right before its int8 GEMM, whose int32
 * accumulators are dequantised ((acc * s_x) * s_w) + b in the epilogue.
 * enable = 0 returns to bf16. dfh_set_weights turns the mode off. */
typedef struct DfhInt8Linear {
  const void* w;       /* int8 [out, in] row-major, device */
  const float* scale;  /* float32 [out], device */
} DfhInt8Linear;
typedef struct DfhInt8Weights {
  DfhInt8Linear input, t_mlp2, d_mlp2;
  DfhInt8Linear ada;                            /* [n_blocks * 6H + 2H, H] */
  const DfhInt8Linear *qkv, *o, *fc1, *fc2;     /* host arrays [n_blocks]; qkv [3H, H] */
} DfhInt8Weights;
int dfh_set_int8(DfhHandle* h, int enable, const DfhInt8Weights* w, void* stream);
/* int8 mode: the LayerNorm + modulate in front of QKV and fc1 also writes its
 * rows per-token quantised (default on), bit-identical to quantising its bf16
 * output in a pass of its own (off). No reference counterpart: in
 * D/int8_dit.py:57-58 the quantisation is part of Int8DynamicLinear.forward;
 * fusing it is a scheduling choice of this library. */
int dfh_set_ln_quant(DfhHandle* h, int enable);

/* dfh_gemm_bf16 with a device workspace (ws, ws_bytes) for the K-split of the
 * last partial round of tiles (see dfh_set_ksplit); too small or NULL: no split.
 * ws_bytes >= 4 * (4096 + 65536 * (number of CUs)) always suffices. The workspace must be
 * zero-filled before its first use; calls leave it reusable (its tile counters
 * return to zero). Calls sharing one workspace must not overlap. */
int dfh_gemm_bf16_ws(const void* A, long lda, const void* B, long ldb, void* C, long ldc,
                     const void* bias, int M, int N, int K, int epilogue, int tile, void* ws, long ws_bytes,
                     void* stream);

/* W8A8 linear (Int8DynamicLinear, int8_dit.py:34-65).
 * Per-row dynamic activation quantisation of bf16 x [M, K] in bf16 arithmetic
 * (int8_dit.py:57-58): q int8 [M, K], scale f32 [M] (bf16 values). */
int dfh_quant_act_i8(const void* x, long ldx, void* q, long ldq, void* scale, int M, int K, void* stream);
/* Per-output-channel weight quantisation in float32 (int8_dit.py:40-45) of bf16
 * W [N, K]: q int8 [N, K] (row-major, K contiguous: the transpose of the
 * reference's Wt_int8 [K, N]), scale f32 [N]. */
int dfh_quant_weight_i8(const void* w, void* q, void* scale, int N, int K, void* stream);
/* acc[m, n] = sum_k xq[m, k] * wq[n, k] in int32 (== torch._int_mm(xq, wq^T)).
 * out_int32 = 1: out int32 [M, N]; else out bf16 = ((acc * sx[m]) * sw[n]) + bias[n]
 * (bias bf16 or NULL). K a multiple of 64; ldx/ldw in bytes, ldo in elements. */
int dfh_gemm_w8a8(const void* xq, long ldx, const void* wq, long ldw, void* out, long ldo, const void* sx,
                  const void* sw, const void* bias, int M, int N, int K, int out_int32, int tile, void* stream);
/* dfh_gemm_w8a8 with a K-split workspace (as dfh_gemm_bf16_ws); int32 sums are exact either way. */
int dfh_gemm_w8a8_ws(const void* xq, long ldx, const void* wq, long ldw, void* out, long ldo, const void* sx,
                     const void* sw, const void* bias, int M, int N, int K, int out_int32, int tile, void* ws,
                     long ws_bytes, void* stream);

/* Prefix K/V cache of a MeanFlow solve (per-(timestep, layer) cache of
 * cached_fm.py:82-197, FMCache / extend_cache / active_forward, restated for the
 * MeanFlow DiT: c_k = T(t_k) + D(dt_k) + g, one branch). Each of n_streams
 * streams holds up to `capacity` rows (prefix + the 1 + P active rows).
 * dfh_kvcache_extend appends counts[i] history rows of stream i (FM sequence
 * space, before input_layer; rows bf16 [n, m_max, H]) at every timestep: they
 * attend causally to the cached prefix and each other (extend_cache).
 * dfh_kvcache_solve runs the NFE-step MeanFlow solve of the active rows — the
 * last hidden row (bf16 [n, H], position = prefix length) and P latent rows —
 * against the cache (active_forward); it equals the full-recompute solve of
 * the sequence prefix + last hidden row. t/dt grids: host [num_steps]. */
int dfh_kvcache_create(DfhHandle* h, int n_streams, int capacity, int num_steps, DfhKVCache** out);
int dfh_kvcache_destroy(DfhKVCache* c);
int dfh_kvcache_reset(DfhKVCache* c, void* stream);
int dfh_kvcache_lengths(DfhKVCache* c, int* lens);
int dfh_kvcache_extend(DfhKVCache* c, const void* rows, int m_max, const int* counts, const void* g_cond,
                       const float* t_grid, const float* dt_grid, void* stream);
int dfh_kvcache_solve(DfhKVCache* c, const void* last_hidden, const void* g_cond, const void* noise, void* out,
                      const float* t_grid, const float* dt_grid, void* stream);

/* Paged KV cache of the LLM backbone (Qwen2.5-1.5B: 12 query heads, 2 KV heads,
 * head_dim 128, 256-token pages).
 *
 * dfh_store_kvcache <- store_kvcache, nanovllm_dots/layers/attention.py:10-47:
 * key / value rows i (D = kv_heads * head_dim bf16, row strides in elements)
 * go to row slot_mapping[i] of k_cache / v_cache ([num_slots, D]); slot -1
 * skips the token. D and the strides multiples of 8, bases 16-B aligned. */
int dfh_store_kvcache(const void* key, long key_stride, const void* value, long value_stride, void* k_cache,
                      void* v_cache, const int* slot_mapping, int n_tokens, int D, void* stream);

/* dfh_paged_attention <- flash_attn_varlen_func (with or without block_table)
 * and flash_attn_with_kvcache (k = v = None) as layers/attention.py:66-95 call
 * them (flash-attn 2.8.3). Sequence i: query tokens cu_seqlens_q[i] ..
 * cu_seqlens_q[i+1] of q, Lk_i keys (cu_seqlens_k diff, or seqlens_k[i] =
 * cache_seqlens). Key t: page block_table[i][t / block_size], offset
 * t % block_size, of k_cache / v_cache [num_blocks, block_size, kv_heads,
 * head_dim]; with block_table NULL, row cu_seqlens_k[i] + t of k / v
 * [total_k, kv_heads, head_dim]. causal: bottom-right aligned (token j of Lq
 * sees keys [0, Lk - Lq + j]); a row that sees no key is written as 0. Query
 * head h reads KV head h / (num_heads / num_kv_heads). out [total_q, num_heads,
 * head_dim] bf16. head_dim 64 or 128; block_size a multiple of 256; q, k, v
 * 16-B aligned, strides (elements between tokens) multiples of 8. The
 * workspace holds dfh_paged_attention_workspace(a) bytes. */
typedef struct DfhPagedAttnArgs {
  int batch, num_heads, num_kv_heads, head_dim;
  int max_seqlen_q, max_seqlen_k;   /* host upper bounds */
  const void* q;
  long q_stride;
  const int* cu_seqlens_q;          /* int32 [batch + 1] device */
  const void* k;
  const void* v;
  long kv_stride;
  const int* cu_seqlens_k;          /* int32 [batch + 1] device, or NULL (then seqlens_k) */
  const int* seqlens_k;             /* int32 [batch] device, or NULL */
  const int* block_table;           /* int32 [batch, block_table_stride] device, or NULL */
  int block_table_stride, block_size;
  void* out;
  long out_stride;
  float softmax_scale;
  int causal;
  void* workspace;                  /* 256-B aligned */
  long workspace_bytes;
  long total_q;                     /* query rows of the batch (q's first dimension), or 0 if unknown:
                                       bounds the row tiles, so the workspace is sized by the batch's
                                       actual rows instead of batch * max_seqlen_q */
} DfhPagedAttnArgs;
long dfh_paged_attention_workspace(const DfhPagedAttnArgs* a);
int dfh_paged_attention(const DfhPagedAttnArgs* a, void* stream);
/* No counterpart in the reference: dfh_paged_attention for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments and results; a->workspace and
 * a->workspace_bytes are ignored and the library's static device scratch is
 * used instead: 64 MiB per GPU, held until the process ends (a decode of 64
 * sequences x 4096 keys, 2 KV heads of head_dim 128, needs 32.5 MiB). Calls whose
 * dfh_paged_attention_workspace(a) exceeds 64 MiB fail with an error. Every
 * call on a GPU shares that GPU's scratch: calls that overlap on one GPU (two
 * streams, or two threads) race. No hipMalloc, hipFree or memset. */
int dfh_paged_attention_noalloc(const DfhPagedAttnArgs* a, void* stream);

/* The patch encoder's per-patch decode (VAESemanticEncoder.decode_patch,
 * nanovllm_dots/models/dots/native/patch_encoder.py:198-215) for n requests at
 * once, request i in cache row rows[i] at that row's own history length:
 * FlashPatchEncoder (nanovllm_dots/models/dots/flash_patch_encoder.py:35-139).
 * A handle owns the packed bf16 weights, per layer a K and a V cache of
 * max_batch rows x capacity tokens x hidden, per row a conv tail (the last
 * latent frame of its previous patch) and a length, and the workspace. Encoder
 * layers: LayerNorm (affine) -> q, k, v without bias -> K / V appended at the
 * row's length -> causal attention over the row's keys -> o_proj -> residual ->
 * LayerNorm -> fc1 -> SiLU -> fc2 -> residual (native/patch_encoder.py:28-85,
 * native/layers.py:210-249). Requirements: hidden a multiple of 256, head_dim
 * 64 or 128, latent_dim a multiple of 32, patch even, out_dim and ffn multiples
 * of 64; capacity is rounded up to a multiple of 256 tokens. */
typedef struct DfhPatchEncConfig {
  int latent_dim, patch, hidden, heads, ffn, n_layers, out_dim;
  int max_batch;                    /* cache rows */
  int capacity;                     /* tokens per row: max patches * patch / 2 */
  float ln_eps;                     /* 1e-5 */
} DfhPatchEncConfig;
/* device bf16 parameters in nn.Linear [out, in] layout (state-dict names
 * encoder.layers.{l}.attn.{q,k,v,o}_proj, attn_norm, ffn_norm, ffn.fc1, ffn.fc2) */
typedef struct DfhPatchEncLayerWeights {
  const void *attn_norm_w, *attn_norm_b, *q_w, *k_w, *v_w, *o_w, *o_b;
  const void *ffn_norm_w, *ffn_norm_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
} DfhPatchEncLayerWeights;
/* ds_w: ds_proj.weight [latent_dim, latent_dim, 2]; in_w: in_proj [hidden,
 * latent_dim]; out_w: out_proj [out_dim, hidden * patch / 2] */
typedef struct DfhPatchEncWeights {
  const void *ds_w, *ds_b, *in_w, *in_b, *out_w, *out_b;
  const DfhPatchEncLayerWeights* layers;   /* host array [n_layers] */
} DfhPatchEncWeights;
typedef struct DfhPatchEnc DfhPatchEnc;
/* <- FlashPatchEncoder.__init__ (flash_patch_encoder.py:43-62): copies the
 * weights, allocates the caches (rows at length 0, zero tails). */
int dfh_patchenc_create(const DfhPatchEncConfig* cfg, const DfhPatchEncWeights* w, DfhPatchEnc** out);
int dfh_patchenc_destroy(DfhPatchEnc* h);
/* <- FlashPatchEncoder.reset_rows (flash_patch_encoder.py:64-69): rows (device
 * int32 [n]) back to length 0 and a zero conv tail. */
int dfh_patchenc_reset_rows(DfhPatchEnc* h, const int* rows, int n, void* stream);
/* <- FlashPatchEncoder.decode_patch (flash_patch_encoder.py:103-139): patches
 * [n, patch, latent_dim] bf16 (row stride patch_stride elements between
 * requests), rows device int32 [n], distinct -> out [n, out_dim] bf16; each
 * row's length advances by patch / 2. A row that would pass its capacity
 * appends nothing and raises the overflow flag of dfh_patchenc_lengths. */
int dfh_patchenc_decode(DfhPatchEnc* h, const void* patches, long patch_stride, const int* rows, int n, void* out,
                        void* stream);
/* lengths of all max_batch rows and the overflow flag (then cleared), copied to
 * the host after the device finishes its queued work (synchronizes) */
int dfh_patchenc_lengths(DfhPatchEnc* h, int* lengths, int* overflow);

#ifdef __cplusplus
}
#endif

#endif /* DOTS_FM_H */
