// rv_quant.hpp — launchers of the quantized-projection kernels (rv_quant.hip),
// called by the validating C ABI in rv_gemv_abi.cpp. Every launcher assumes
// its arguments were validated: lengths, formats and 4-byte alignment.
#pragma once

#include "../../include/ramvamp_gemv.h"
#include "rv_internal.hpp"

namespace rv {

// The fused projections (one launch): up to three row ranges of
// independent matrices, each against the Q8_K (k-quant formats) or the Q8_0
// (RV_QF_Q8_0) form of one f32 activation row x, which each workgroup
// quantizes into LDS before its rows run. x holds nbk * 256 = nb0 * 32
// values, at most kFusedMaxKBlocks * 256.
constexpr int kFusedWaves = 8;
constexpr int kFusedMaxKBlocks = 32;
constexpr int kFusedMax0Blocks = kFusedMaxKBlocks * 8;
// With norm_w set, x is first RMS-normalized (norm.rs:18-58: f64 mean of
// squares, x * inv * w in f32) in LDS, and the normalized row is what gets
// quantized. With a segment's `add` set, its rows store add[i] + dot
// (vec.rs:10-22; add may alias out).
struct FusedSeg {
  uint32_t fmt;
  const uint8_t* w;
  size_t row_bytes;
  float* out;
  const float* add;
};
struct FusedProjArgs {
  const float* x;
  int nbk, nb0;
  int n_seg;
  FusedSeg seg[3];
  int n_rows[3];
  const float* norm_w;
  float eps;
  // Optional: a token graph's device position; above gate_max the launch
  // writes nothing (its decode step was refused).
  const uint32_t* gate_pos;
  uint32_t gate_max;
};

// The attention projections of one token (forward.rs:2574-2646) as the C
// ABI and the fused attention block use them: validation (check, fills the
// row sizes) apart from the launches, so a composite call can validate
// everything before it launches anything.
struct InProj {
  const float* x;       // the normed row, or with norm_w the row to normalize
  const float* norm_w;  // optional: RMSNorm weight [hidden], applied first
  float eps;
  size_t hidden;
  uint32_t q_format;
  const uint8_t* wq;
  size_t rb_q;
  float* q;
  size_t q_dim;
  const uint8_t* wk;
  size_t rb_k;
  float* k;
  size_t kv_dim;
  uint32_t v_format;
  const uint8_t* wv;
  size_t rb_v;
  float* v;
  void* scratch;     // in_proj_scratch_bytes(hidden, norm_w != nullptr) bytes
};
struct OutProj {
  const float* x;    // attn_out [q_dim]
  size_t q_dim;
  uint32_t o_format;
  const uint8_t* wo;
  size_t rb;
  float* o;          // [hidden]
  size_t hidden;
  bool add;          // o[i] += dot (the residual add) instead of o[i] = dot
  void* scratch;     // out_proj_scratch_bytes(q_dim, hidden, add) bytes
  // Optional (fused launch only): nothing is written when *gate_pos >
  // gate_max (a token graph's refused decode step).
  const uint32_t* gate_pos = nullptr;
  uint32_t gate_max = 0;
};
size_t in_proj_scratch_bytes(size_t hidden, bool norm);
size_t out_proj_scratch_bytes(size_t q_dim, size_t hidden, bool add);
int32_t in_proj_check(InProj& p, size_t wq_len, size_t wk_len, size_t wv_len, rv_error* err);
int32_t out_proj_check(OutProj& p, size_t wo_len, rv_error* err);
HipStatus in_proj_launch(const InProj& p, hipStream_t s);
HipStatus out_proj_launch(const OutProj& p, hipStream_t s);
// The same for n_rows rows of a prefill chunk (prefill.rs:1985-2053,
// :2113-2154): x and the outputs row-major; the out form adds into o (the
// residual rows). p.scratch holds the rows' quantized blocks.
size_t in_proj_rows_scratch_bytes(size_t n_rows, size_t hidden);
size_t out_proj_rows_scratch_bytes(size_t n_rows, size_t q_dim);
int32_t in_proj_rows_check(InProj& p, size_t n_rows, size_t wq_len, size_t wk_len, size_t wv_len, rv_error* err);
int32_t out_proj_rows_check(OutProj& p, size_t n_rows, size_t wo_len, rv_error* err);
HipStatus in_proj_rows_launch(const InProj& p, size_t n_rows, hipStream_t s);
HipStatus out_proj_rows_launch(const OutProj& p, size_t n_rows, hipStream_t s);
// out[r] = rmsnorm(x[r], w, eps), n_rows rows of n values.
HipStatus launch_rmsnorm_rows(const float* x, const float* w, float eps, size_t n_rows, size_t n, float* out,
                              hipStream_t s);

HipStatus launch_quantize_q8_k(const float* x, rv_block_q8_k* out, size_t n_blocks, hipStream_t s);
HipStatus launch_quantize_q8_0(const float* x, rv_block_q8_0* out, size_t n_blocks, hipStream_t s);
// Both forms of n_k_blocks * 256 values in one launch (Q8_K blocks to ok,
// 8 n_k_blocks Q8_0 blocks to o0).
HipStatus launch_quantize_both(const float* x, rv_block_q8_k* ok, rv_block_q8_0* o0, size_t n_k_blocks,
                               hipStream_t s);
// out[i] = row(row_lo + i) . acts, i < n_rows; acts quantized blocks
// (Q8_K, or Q8_0 for RV_QF_Q8_0) in global memory.
HipStatus launch_gemv_rows(uint32_t fmt, const uint8_t* w, size_t row_bytes, size_t in_dim, const void* acts,
                           size_t row_lo, size_t n_rows, float* out, hipStream_t s);
HipStatus launch_fused_proj(const FusedProjArgs& a, hipStream_t s);
// Batched GEMV (int8 MFMA): out[i * ldo + a] (or, transposed, out[a * ldo + i])
// = row(row_lo + i) . act_row(a), i < n_rows, a < n_acts; acts holds n_acts
// rows of in_dim / 256 Q8_K (or in_dim / 32 Q8_0 for RV_QF_Q8_0) blocks.
// in_dim > 0. With accumulate, out += the dot instead.
HipStatus launch_gemv_batched(uint32_t fmt, const uint8_t* w, size_t row_bytes, size_t in_dim, const void* acts,
                              size_t n_acts, size_t row_lo, size_t n_rows, float* out, size_t ldo, bool transposed,
                              hipStream_t s, bool accumulate = false);
// out = rmsnorm(x, w, eps) over n values (one workgroup; norm.rs:38-58).
HipStatus launch_rmsnorm(const float* x, const float* w, float eps, size_t n, float* out, hipStream_t s);
// a[i] += b[i], i < n (vec.rs:10-22).
HipStatus launch_vec_add(float* a, const float* b, size_t n, hipStream_t s);
// out[0 .. n) = 0 (a kernel, so the call can be captured into a graph).
HipStatus launch_fill_zero(float* out, size_t n, hipStream_t s);

}  // namespace rv
