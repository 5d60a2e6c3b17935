// Host launchers of the row / elementwise kernels (internal to the library).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dfh_kernels.h"

namespace dfh {

constexpr int kMaxTimeVals = 16;
struct TimeVals {
  float v[kMaxTimeVals];
};

// Request layout from pos_ids (padded inputs) or from lens (varlen inputs).
// Optional: tail_seqs [n] (the P latent queries of each request, output rows
// i*P + j), tail_req [n*P] and tail_pos [n*P] (request and position of compact
// latent row i*P + j).
hipError_t fm_layout(const float* pos_ids, const int* lens, int n, int T, int P, int* cu_rows, int* cu_vt,
                     int* hist_len, int* counts, int* err, AttnSeq* seqs, AttnSeq* tail_seqs, int* tail_req,
                     int* tail_pos, hipStream_t s);
hipError_t prefix_tables(const uint16_t* rows_in, long stride_in, int m_max, int H, const int* counts,
                         const int* lens, const int* offs, int n, int S, int cap, uint16_t* seq, int* row_req,
                         int* row_pos, int* c_rows, int* vt_col, AttnSeq* seqs, hipStream_t s);
hipError_t active_tables(const int* lens, int n, int S, int P, int cap, int* row_req, int* row_pos,
                         int* c_rows, int* vt_col, AttnSeq* seqs, int* patch_rows, int* lh_rows,
                         hipStream_t s);
hipError_t cache_advance(int* lens, const int* counts, int n, hipStream_t s);
// Rows from the padded input inp [n, T, H], or (inp NULL) from per-request
// history bases src_rows[i] (device array of device pointers), row stride src_stride
hipError_t fm_gather(const uint16_t* inp, const uint16_t* const* src_rows, long src_stride, int n, int T,
                     int P, int H, const int* cu_rows, const int* cu_vt, const int* hist_len, uint16_t* seq,
                     int* row_req, int* row_pos, int* vt_col, int* patch_rows, int* err, hipStream_t s);
// cos / sin of pos * inv_freq[d] (float32) for half = 32, positions grouped by 32
// (rope_table_kernel); the tables hold ceil(max_pos / 32) * 32 * 32 floats
hipError_t rope_table(const float* inv_freq, int half, int max_pos, float* cosv, float* sinv,
                      hipStream_t s);
hipError_t timestep_embed(const float* tv, const TimeVals& tvh, int rows, const float* freqs, int half,
                          int dim, uint16_t* out, hipStream_t s);
hipError_t silu_bf16(const uint16_t* x, uint16_t* y, long n, hipStream_t s);
hipError_t condition(const uint16_t* temb, const uint16_t* demb, const uint16_t* g, int S, int N,
                     int H, uint16_t* c_out, uint16_t* a_out, hipStream_t s, bool per_request_t);
hipError_t unpack_rows(const uint16_t* src, int n, int T, int P, int D, const int* cu_rows,
                       const int* hist_len, uint16_t* dst, hipStream_t s);
hipError_t scatter_rows(const uint16_t* src, const int* rows_idx, int rows, int H, uint16_t* dst,
                        hipStream_t s);
// dst row (dst_rows ? dst_rows[r] : r) = src row (src_rows ? src_rows[r] : r), r < rows
hipError_t gather_rows(const uint16_t* src, const int* src_rows, const int* dst_rows, int rows, int H,
                       uint16_t* dst, hipStream_t s);
hipError_t z_update(uint16_t* z, const uint16_t* v, float dt, long n, hipStream_t s);

// patch encoder (patch_encoder.hip)
hipError_t ln_affine(const uint16_t* x, uint16_t* out, const uint16_t* w, const uint16_t* b, int rows, int H,
                     float eps, hipStream_t s);
hipError_t pe_downsample(const uint16_t* patch, long patch_stride, const uint16_t* w, const uint16_t* bias,
                         const int* rows, uint16_t* tail, uint16_t* out, int n, int P, int ld, hipStream_t s);
hipError_t pe_plan(const int* rows, const int* len, int n, int ods, int cap, int max_rows, int* rows_ok, int* slots,
                   int* seqlens_k, int* cu_q, int* err, hipStream_t s);
hipError_t pe_advance(const int* rows, int* len, int n, int ods, int cap, hipStream_t s);
hipError_t pe_reset(const int* rows, int n, int max_rows, int* len, uint16_t* tail, int ld, hipStream_t s);

}  // namespace dfh
