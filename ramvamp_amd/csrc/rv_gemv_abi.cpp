// rv_gemv_abi.cpp — the C ABI of the quantized projections (include/ramvamp_gemv.h).
//
// Host-side validation in the reference's order, then the launches in
// rv_quant.hip. Mirrors kernels/quants/quantize.rs (check_len, :11-26),
// kernels/gemv.rs (`validate`, :212-266; `k_quant_dot`, :268-279) and the
// per-layer call sequence of model/forward.rs:2574-2646.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <limits>

#include "rv_quant.hpp"

namespace {

int32_t fail(rv_error* err, int32_t code, uint64_t a, uint64_t b, uint64_t c, const char* what) {
  if (err) {
    err->code = code;
    err->a = a;
    err->b = b;
    err->c = c;
    err->d = 0;
    err->what = what;
  }
  return code;
}

int32_t ok(rv_error* err) {
  if (err) *err = rv_error{RV_OK, 0, 0, 0, 0, nullptr};
  return RV_OK;
}

size_t sat_mul(size_t a, size_t b) {
  size_t r;
  return __builtin_mul_overflow(a, b, &r) ? std::numeric_limits<size_t>::max() : r;
}

bool aligned4(const void* p) { return ((uintptr_t)p & 3) == 0; }

int32_t check_flags(uint32_t flags, rv_error* err) {
  if (flags & RV_HOST_PTRS) return fail(err, RV_ERR_UNSUPPORTED, flags, 0, 0, "RV_HOST_PTRS (device pointers only)");
  return RV_OK;
}

int32_t finish(hipStream_t s, uint32_t flags, const rv::HipStatus& st, rv_error* err) {
  if (st.e != hipSuccess) return fail(err, RV_ERR_HIP, (uint64_t)st.e, 0, 0, st.what);
  if (flags & RV_SYNC) {
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(err, RV_ERR_HIP, (uint64_t)e, 0, 0, "hipStreamSynchronize");
  }
  return ok(err);
}

bool k_quant(uint32_t f) { return f == RV_QF_Q4_K || f == RV_QF_Q5_K || f == RV_QF_Q6_K; }

// quantize.rs check_len (:11-26).
int32_t check_quantize(uint32_t format, size_t floats, size_t out_blocks, rv_error* err) {
  const size_t width = format == RV_QF_Q8_0 ? 32 : 256;
  if (floats != sat_mul(out_blocks, width))
    return fail(err, RV_QUANT_QUANTIZE_LEN_MISMATCH, format, floats, out_blocks, "quantize");
  return RV_OK;
}

// gemv.rs `validate` (:212-266); returns row_bytes. The products with
// n_acts saturate, so an absurd n_acts falls out as a mismatch.
int32_t check_gemv(const char* what, uint32_t format, size_t weight_len, size_t in_dim, size_t out_dim,
                   size_t act_blocks, size_t row_lo, size_t row_hi, size_t out_len, size_t* row_bytes, rv_error* err,
                   size_t n_acts = 1) {
  const int32_t rc = rv_quant_row_bytes(format, in_dim, row_bytes, err);
  if (rc) return rc;
  const size_t expected = sat_mul(*row_bytes, out_dim);
  if (expected != weight_len) return fail(err, RV_PRIM_LENGTH_MISMATCH, weight_len, expected, 0, what);
  if (row_lo > row_hi)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, row_lo, row_hi, 0, "gemv rows: row range start vs end");
  if (row_hi > out_dim)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, row_hi, out_dim, 0, "gemv rows: row range end vs out_dim");
  const size_t wanted = sat_mul(row_hi - row_lo, n_acts);
  if (out_len != wanted) return fail(err, RV_PRIM_LENGTH_MISMATCH, out_len, wanted, 0, what);
  const size_t wb = sat_mul(in_dim / rv_quant_block_weights(format), n_acts);
  if (wb != act_blocks) return fail(err, RV_QUANT_BLOCK_COUNT_MISMATCH, wb, act_blocks, 0, "gemv");
  return RV_OK;
}

int32_t check_ptrs(rv_error* err, std::initializer_list<std::pair<const void*, const char*>> ps) {
  for (const auto& p : ps) {
    if (!p.first) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, p.second);
    if (!aligned4(p.first)) return fail(err, RV_ERR_UNSUPPORTED, (uintptr_t)p.first, 0, 0, "pointer not 4-byte aligned");
  }
  return RV_OK;
}

size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

// An empty row range writes nothing; rows of no weights are empty sums, 0.
int32_t empty_rows(float* out, size_t n, void* stream, uint32_t flags, rv_error* err) {
  const hipStream_t s = (hipStream_t)stream;
  if (n == 0) return finish(s, flags, rv::HipStatus{}, err);
  if (!out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, "out");
  return finish(s, flags, rv::launch_fill_zero(out, n, s), err);
}

}  // namespace

extern "C" {

size_t rv_quant_block_weights(uint32_t format) {
  switch (format) {
    case RV_QF_Q4_K:
    case RV_QF_Q5_K:
    case RV_QF_Q6_K:
    case RV_QF_Q8_K: return 256;
    case RV_QF_Q8_0: return 32;
    default: return 0;
  }
}

size_t rv_quant_block_bytes(uint32_t format) {
  switch (format) {
    case RV_QF_Q4_K: return 144;
    case RV_QF_Q5_K: return 176;
    case RV_QF_Q6_K: return 210;
    case RV_QF_Q8_0: return 34;
    case RV_QF_Q8_K: return 292;
    default: return 0;
  }
}

int32_t rv_quant_row_bytes(uint32_t format, size_t in_dim, size_t* row_bytes, rv_error* err) {
  if (!row_bytes) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, "row_bytes");
  const size_t bw = rv_quant_block_weights(format);
  if (!bw) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "row_bytes");
  if (in_dim % bw) return fail(err, RV_QUANT_INDIVISIBLE_ROW, format, in_dim, bw, "row_bytes");
  *row_bytes = in_dim / bw * rv_quant_block_bytes(format);
  return ok(err);
}

int32_t rv_quantize_row_q8_0(const float* x, size_t x_len, rv_block_q8_0* out, size_t n_blocks, void* stream,
                             uint32_t flags, rv_error* err) {
  int32_t rc = check_quantize(RV_QF_Q8_0, x_len, n_blocks, err);
  if (rc || (rc = check_flags(flags, err))) return rc;
  if (n_blocks == 0) return ok(err);
  if ((rc = check_ptrs(err, {{x, "x"}, {out, "out"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::launch_quantize_q8_0(x, out, n_blocks, s), err);
}

int32_t rv_quantize_row_q8_k(const float* x, size_t x_len, rv_block_q8_k* out, size_t n_blocks, void* stream,
                             uint32_t flags, rv_error* err) {
  int32_t rc = check_quantize(RV_QF_Q8_K, x_len, n_blocks, err);
  if (rc || (rc = check_flags(flags, err))) return rc;
  if (n_blocks == 0) return ok(err);
  if ((rc = check_ptrs(err, {{x, "x"}, {out, "out"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::launch_quantize_q8_k(x, out, n_blocks, s), err);
}

int32_t rv_gemv_q8_k_rows(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                          const rv_block_q8_k* acts, size_t act_blocks, size_t row_lo, size_t row_hi, float* out,
                          size_t out_len, void* stream, uint32_t flags, rv_error* err) {
  if (!k_quant(format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "gemv_q8_k_rows");
  size_t row_bytes;
  int32_t rc = check_gemv("gemv_q8_k_rows: weight bytes vs rows / out vs range", format, weight_len, in_dim, out_dim,
                          act_blocks, row_lo, row_hi, out_len, &row_bytes, err);
  if (rc || (rc = check_flags(flags, err))) return rc;
  if (row_hi == row_lo || in_dim == 0) return empty_rows(out, row_hi - row_lo, stream, flags, err);
  if ((rc = check_ptrs(err, {{weight, "weight"}, {acts, "acts"}, {out, "out"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::launch_gemv_rows(format, weight, row_bytes, in_dim, acts, row_lo, row_hi - row_lo, out, s),
                err);
}

int32_t rv_gemv_q8_k(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                     const rv_block_q8_k* acts, size_t act_blocks, float* out, size_t out_len, void* stream,
                     uint32_t flags, rv_error* err) {
  if (!k_quant(format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "gemv_q8_k");
  return rv_gemv_q8_k_rows(format, weight, weight_len, in_dim, out_dim, acts, act_blocks, 0, out_dim, out, out_len,
                           stream, flags, err);
}

int32_t rv_gemv_q8_0_rows(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                          const rv_block_q8_0* acts, size_t act_blocks, size_t row_lo, size_t row_hi, float* out,
                          size_t out_len, void* stream, uint32_t flags, rv_error* err) {
  size_t row_bytes;
  int32_t rc = check_gemv("gemv_q8_0_rows: weight bytes vs rows / out vs range", RV_QF_Q8_0, weight_len, in_dim,
                          out_dim, act_blocks, row_lo, row_hi, out_len, &row_bytes, err);
  if (rc || (rc = check_flags(flags, err))) return rc;
  if (row_hi == row_lo || in_dim == 0) return empty_rows(out, row_hi - row_lo, stream, flags, err);
  if ((rc = check_ptrs(err, {{weight, "weight"}, {acts, "acts"}, {out, "out"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags,
                rv::launch_gemv_rows(RV_QF_Q8_0, weight, row_bytes, in_dim, acts, row_lo, row_hi - row_lo, out, s),
                err);
}

int32_t rv_gemv_q8_0(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                     const rv_block_q8_0* acts, size_t act_blocks, float* out, size_t out_len, void* stream,
                     uint32_t flags, rv_error* err) {
  return rv_gemv_q8_0_rows(weight, weight_len, in_dim, out_dim, acts, act_blocks, 0, out_dim, out, out_len, stream,
                           flags, err);
}

int32_t rv_gemv_q8_k_batched(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim,
                             size_t out_dim, const rv_block_q8_k* acts, size_t act_blocks, size_t n_acts,
                             size_t row_lo, size_t row_hi, float* out, size_t out_len, void* stream, uint32_t flags,
                             rv_error* err) {
  if (!k_quant(format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "gemv_q8_k_batched");
  size_t row_bytes;
  int32_t rc = check_gemv("gemv_q8_k_batched: weight bytes vs rows / out vs range x n_acts", format, weight_len,
                          in_dim, out_dim, act_blocks, row_lo, row_hi, out_len, &row_bytes, err, n_acts);
  if (rc || (rc = check_flags(flags, err))) return rc;
  if (out_len == 0 || in_dim == 0) return empty_rows(out, out_len, stream, flags, err);
  if ((rc = check_ptrs(err, {{weight, "weight"}, {acts, "acts"}, {out, "out"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags,
                rv::launch_gemv_batched(format, weight, row_bytes, in_dim, acts, n_acts, row_lo, row_hi - row_lo, out,
                                        n_acts, false, s),
                err);
}

int32_t rv_gemv_q8_0_batched(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                             const rv_block_q8_0* acts, size_t act_blocks, size_t n_acts, size_t row_lo,
                             size_t row_hi, float* out, size_t out_len, void* stream, uint32_t flags, rv_error* err) {
  size_t row_bytes;
  int32_t rc = check_gemv("gemv_q8_0_batched: weight bytes vs rows / out vs range x n_acts", RV_QF_Q8_0, weight_len,
                          in_dim, out_dim, act_blocks, row_lo, row_hi, out_len, &row_bytes, err, n_acts);
  if (rc || (rc = check_flags(flags, err))) return rc;
  if (out_len == 0 || in_dim == 0) return empty_rows(out, out_len, stream, flags, err);
  if ((rc = check_ptrs(err, {{weight, "weight"}, {acts, "acts"}, {out, "out"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags,
                rv::launch_gemv_batched(RV_QF_Q8_0, weight, row_bytes, in_dim, acts, n_acts, row_lo,
                                        row_hi - row_lo, out, n_acts, false, s),
                err);
}

size_t rv_attn_in_proj_rows_scratch_bytes(size_t n_rows, size_t hidden) {
  return rv::in_proj_rows_scratch_bytes(n_rows, hidden);
}

int32_t rv_attn_in_proj_rows(const float* normed_rows, size_t n_rows, size_t hidden, uint32_t q_format,
                             const uint8_t* wq, size_t wq_len, float* q_rows, size_t q_dim, const uint8_t* wk,
                             size_t wk_len, float* k_rows, size_t kv_dim, uint32_t v_format, const uint8_t* wv,
                             size_t wv_len, float* v_rows, void* scratch, size_t scratch_len, void* stream,
                             uint32_t flags, rv_error* err) {
  rv::InProj p{normed_rows, nullptr, 0.f, hidden, q_format, wq, 0, q_rows, q_dim, wk, 0, k_rows, kv_dim,
               v_format, wv, 0, v_rows, scratch};
  int32_t rc;
  if ((rc = rv::in_proj_rows_check(p, n_rows, wq_len, wk_len, wv_len, err))) return rc;
  const size_t need = rv_attn_in_proj_rows_scratch_bytes(n_rows, hidden);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, 0, "attn_in_proj_rows scratch");
  if ((rc = check_flags(flags, err))) return rc;
  if (n_rows == 0) return finish((hipStream_t)stream, flags, rv::HipStatus{}, err);
  if (hidden == 0) return fail(err, RV_ERR_UNSUPPORTED, 0, 0, 0, "attn_in_proj_rows with hidden 0");
  if ((rc = check_ptrs(err, {{normed_rows, "normed_rows"}, {wq, "wq"}, {q_rows, "q_rows"}, {wk, "wk"},
                             {k_rows, "k_rows"}, {wv, "wv"}, {v_rows, "v_rows"}, {scratch, "scratch"}})))
    return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::in_proj_rows_launch(p, n_rows, s), err);
}

size_t rv_attn_out_proj_rows_scratch_bytes(size_t n_rows, size_t q_dim) {
  return rv::out_proj_rows_scratch_bytes(n_rows, q_dim);
}

int32_t rv_attn_out_proj_rows(const float* attn_rows, size_t n_rows, size_t q_dim, uint32_t o_format,
                              const uint8_t* wo, size_t wo_len, float* residual_rows, size_t hidden, void* scratch,
                              size_t scratch_len, void* stream, uint32_t flags, rv_error* err) {
  rv::OutProj p{attn_rows, q_dim, o_format, wo, 0, residual_rows, hidden, true, scratch};
  int32_t rc;
  if ((rc = rv::out_proj_rows_check(p, n_rows, wo_len, err))) return rc;
  const size_t need = rv_attn_out_proj_rows_scratch_bytes(n_rows, q_dim);
  if (scratch_len < need)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, 0, "attn_out_proj_rows scratch");
  if ((rc = check_flags(flags, err))) return rc;
  if (n_rows == 0 || hidden == 0) return finish((hipStream_t)stream, flags, rv::HipStatus{}, err);
  if (q_dim == 0) return fail(err, RV_ERR_UNSUPPORTED, 0, 0, 0, "attn_out_proj_rows with q_dim 0");
  if ((rc = check_ptrs(err, {{attn_rows, "attn_rows"}, {wo, "wo"}, {residual_rows, "residual_rows"},
                             {scratch, "scratch"}})))
    return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::out_proj_rows_launch(p, n_rows, s), err);
}

size_t rv_attn_in_proj_scratch_bytes(size_t hidden) { return rv::in_proj_scratch_bytes(hidden, false); }

int32_t rv_attn_in_proj(const float* normed, size_t hidden, uint32_t q_format, const uint8_t* wq, size_t wq_len,
                        float* q, size_t q_dim, const uint8_t* wk, size_t wk_len, float* k, size_t kv_dim,
                        uint32_t v_format, const uint8_t* wv, size_t wv_len, float* v, void* scratch,
                        size_t scratch_len, void* stream, uint32_t flags, rv_error* err) {
  rv::InProj p{normed, nullptr, 0.f, hidden, q_format, wq, 0, q, q_dim, wk, 0, k, kv_dim, v_format, wv, 0, v, scratch};
  int32_t rc;
  if ((rc = rv::in_proj_check(p, wq_len, wk_len, wv_len, err))) return rc;
  const size_t need = rv_attn_in_proj_scratch_bytes(hidden);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, 0, "attn_in_proj scratch");
  if ((rc = check_flags(flags, err))) return rc;
  if (hidden == 0) return fail(err, RV_ERR_UNSUPPORTED, 0, 0, 0, "attn_in_proj with hidden 0");
  if ((rc = check_ptrs(err, {{normed, "normed"}, {wq, "wq"}, {q, "q"}, {wk, "wk"}, {k, "k"}, {wv, "wv"}, {v, "v"},
                             {scratch, "scratch"}})))
    return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::in_proj_launch(p, s), err);
}

size_t rv_attn_out_proj_scratch_bytes(size_t q_dim) { return rv::out_proj_scratch_bytes(q_dim, 0, false); }

int32_t rv_attn_out_proj(const float* attn_out, size_t q_dim, uint32_t o_format, const uint8_t* wo, size_t wo_len,
                         float* o, size_t hidden, void* scratch, size_t scratch_len, void* stream, uint32_t flags,
                         rv_error* err) {
  rv::OutProj p{attn_out, q_dim, o_format, wo, 0, o, hidden, false, scratch};
  int32_t rc;
  if ((rc = rv::out_proj_check(p, wo_len, err))) return rc;
  const size_t need = rv_attn_out_proj_scratch_bytes(q_dim);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, 0, "attn_out_proj scratch");
  if ((rc = check_flags(flags, err))) return rc;
  if (q_dim == 0) return fail(err, RV_ERR_UNSUPPORTED, 0, 0, 0, "attn_out_proj with q_dim 0");
  if ((rc = check_ptrs(err, {{attn_out, "attn_out"}, {wo, "wo"}, {o, "o"}, {scratch, "scratch"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  return finish(s, flags, rv::out_proj_launch(p, s), err);
}

}  // extern "C"

namespace rv {

size_t in_proj_scratch_bytes(size_t hidden, bool norm) {
  // Rows past the fused limit: the Q8_K and Q8_0 forms of the row (and, with
  // the norm, the normalized row before them).
  const size_t acts = align16(hidden / 256 * sizeof(rv_block_q8_k)) + align16(hidden / 32 * sizeof(rv_block_q8_0));
  return acts + (norm ? hidden * sizeof(float) : 0);
}

size_t out_proj_scratch_bytes(size_t q_dim, size_t hidden, bool add) {
  return align16(q_dim / 256 * sizeof(rv_block_q8_k)) + (add ? hidden * sizeof(float) : 0);
}

int32_t in_proj_check(InProj& p, size_t wq_len, size_t wk_len, size_t wv_len, rv_error* err) {
  // forward.rs:2576-2612 in order: both quantizations, then q, k, v.
  int32_t rc;
  if ((rc = check_quantize(RV_QF_Q8_K, p.hidden, p.hidden / 256, err))) return rc;
  if ((rc = check_quantize(RV_QF_Q8_0, p.hidden, p.hidden / 32, err))) return rc;
  if (!k_quant(p.q_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, p.q_format, 0, 0, "attn_in_proj q");
  if ((rc = check_gemv("attn_in_proj q: weight bytes vs rows / out vs range", p.q_format, wq_len, p.hidden, p.q_dim,
                       p.hidden / 256, 0, p.q_dim, p.q_dim, &p.rb_q, err)))
    return rc;
  if ((rc = check_gemv("attn_in_proj k: weight bytes vs rows / out vs range", RV_QF_Q8_0, wk_len, p.hidden, p.kv_dim,
                       p.hidden / 32, 0, p.kv_dim, p.kv_dim, &p.rb_k, err)))
    return rc;
  if (!k_quant(p.v_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, p.v_format, 0, 0, "attn_in_proj v");
  return check_gemv("attn_in_proj v: weight bytes vs rows / out vs range", p.v_format, wv_len, p.hidden, p.kv_dim,
                    p.hidden / 256, 0, p.kv_dim, p.kv_dim, &p.rb_v, err);
}

int32_t out_proj_check(OutProj& p, size_t wo_len, rv_error* err) {
  // forward.rs:2630-2646: quantize_row_q8_k(attn_out), then the o_proj GEMV.
  int32_t rc;
  if ((rc = check_quantize(RV_QF_Q8_K, p.q_dim, p.q_dim / 256, err))) return rc;
  if (!k_quant(p.o_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, p.o_format, 0, 0, "attn_out_proj");
  return check_gemv("attn_out_proj: weight bytes vs rows / out vs range", p.o_format, wo_len, p.q_dim, p.hidden,
                    p.q_dim / 256, 0, p.hidden, p.hidden, &p.rb, err);
}

HipStatus in_proj_launch(const InProj& p, hipStream_t s) {
  if (p.hidden / 256 <= (size_t)kFusedMaxKBlocks) {
    // One launch: each workgroup (normalizes and) quantizes the row into LDS
    // (both forms, bit-identical to quantize_row_q8_k / _q8_0) and runs its
    // rows; the quantized row never goes through memory and `scratch` is
    // left untouched.
    FusedProjArgs a{};
    a.x = p.x;
    a.nbk = (int)(p.hidden / 256);
    a.nb0 = (int)(p.hidden / 32);
    a.n_seg = 3;
    a.seg[0] = {p.q_format, p.wq, p.rb_q, p.q, nullptr};
    a.seg[1] = {RV_QF_Q8_0, p.wk, p.rb_k, p.k, nullptr};
    a.seg[2] = {p.v_format, p.wv, p.rb_v, p.v, nullptr};
    a.n_rows[0] = (int)p.q_dim;
    a.n_rows[1] = (int)p.kv_dim;
    a.n_rows[2] = (int)p.kv_dim;
    a.norm_w = p.norm_w;
    a.eps = p.eps;
    return launch_fused_proj(a, s);
  }
  // Wider rows: (normalized and) quantized into `scratch`, then the GEMVs.
  auto* acts_k = reinterpret_cast<rv_block_q8_k*>(p.scratch);
  char* next = (char*)p.scratch + align16(p.hidden / 256 * sizeof(rv_block_q8_k));
  auto* acts_0 = reinterpret_cast<rv_block_q8_0*>(next);
  next += align16(p.hidden / 32 * sizeof(rv_block_q8_0));
  HipStatus st;
  const float* x = p.x;
  if (p.norm_w) {
    float* normed = reinterpret_cast<float*>(next);
    st = launch_rmsnorm(p.x, p.norm_w, p.eps, p.hidden, normed, s);
    x = normed;
  }
  if (st.e == hipSuccess) st = launch_quantize_both(x, acts_k, acts_0, p.hidden / 256, s);
  if (st.e == hipSuccess) st = launch_gemv_rows(p.q_format, p.wq, p.rb_q, p.hidden, acts_k, 0, p.q_dim, p.q, s);
  if (st.e == hipSuccess) st = launch_gemv_rows(RV_QF_Q8_0, p.wk, p.rb_k, p.hidden, acts_0, 0, p.kv_dim, p.k, s);
  if (st.e == hipSuccess) st = launch_gemv_rows(p.v_format, p.wv, p.rb_v, p.hidden, acts_k, 0, p.kv_dim, p.v, s);
  return st;
}

HipStatus out_proj_launch(const OutProj& p, hipStream_t s) {
  if (p.q_dim / 256 <= (size_t)kFusedMaxKBlocks) {
    FusedProjArgs a{};
    a.x = p.x;
    a.nbk = (int)(p.q_dim / 256);
    a.nb0 = (int)(p.q_dim / 32);
    a.n_seg = 1;
    a.seg[0] = {p.o_format, p.wo, p.rb, p.o, p.add ? p.o : nullptr};
    a.n_rows[0] = (int)p.hidden;
    a.gate_pos = p.gate_pos;
    a.gate_max = p.gate_max;
    return launch_fused_proj(a, s);
  }
  if (p.gate_pos) {
    HipStatus st;
    st.e = hipErrorNotSupported;
    st.what = "a device-position gate needs the fused output projection (q_dim <= 8192)";
    return st;
  }
  auto* acts = reinterpret_cast<rv_block_q8_k*>(p.scratch);
  float* dst = p.add ? reinterpret_cast<float*>((char*)p.scratch + align16(p.q_dim / 256 * sizeof(rv_block_q8_k)))
                     : p.o;
  HipStatus st = launch_quantize_q8_k(p.x, acts, p.q_dim / 256, s);
  if (st.e == hipSuccess) st = launch_gemv_rows(p.o_format, p.wo, p.rb, p.q_dim, acts, 0, p.hidden, dst, s);
  if (st.e == hipSuccess && p.add) st = launch_vec_add(p.o, dst, p.hidden, s);
  return st;
}

size_t in_proj_rows_scratch_bytes(size_t n_rows, size_t hidden) {
  return align16(sat_mul(n_rows, hidden / 256 * sizeof(rv_block_q8_k))) +
         sat_mul(n_rows, hidden / 32 * sizeof(rv_block_q8_0));
}

size_t out_proj_rows_scratch_bytes(size_t n_rows, size_t q_dim) {
  return sat_mul(n_rows, q_dim / 256 * sizeof(rv_block_q8_k));
}

int32_t in_proj_rows_check(InProj& p, size_t n, size_t wq_len, size_t wk_len, size_t wv_len, rv_error* err) {
  // prefill.rs:1985-2053 in order: each row quantized both ways, then the
  // batched q, k and v projections (their transposes are the store layout).
  int32_t rc;
  if ((rc = check_quantize(RV_QF_Q8_K, p.hidden, p.hidden / 256, err))) return rc;
  if ((rc = check_quantize(RV_QF_Q8_0, p.hidden, p.hidden / 32, err))) return rc;
  if (!k_quant(p.q_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, p.q_format, 0, 0, "gemv_q8_k_batched");
  if ((rc = check_gemv("attn_in_proj_rows q: weight bytes vs rows / out vs range x n_acts", p.q_format, wq_len,
                       p.hidden, p.q_dim, sat_mul(n, p.hidden / 256), 0, p.q_dim, sat_mul(p.q_dim, n), &p.rb_q, err,
                       n)))
    return rc;
  if ((rc = check_gemv("attn_in_proj_rows k: weight bytes vs rows / out vs range x n_acts", RV_QF_Q8_0, wk_len,
                       p.hidden, p.kv_dim, sat_mul(n, p.hidden / 32), 0, p.kv_dim, sat_mul(p.kv_dim, n), &p.rb_k, err,
                       n)))
    return rc;
  if (!k_quant(p.v_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, p.v_format, 0, 0, "gemv_q8_k_batched");
  return check_gemv("attn_in_proj_rows v: weight bytes vs rows / out vs range x n_acts", p.v_format, wv_len, p.hidden,
                    p.kv_dim, sat_mul(n, p.hidden / 256), 0, p.kv_dim, sat_mul(p.kv_dim, n), &p.rb_v, err, n);
}

int32_t out_proj_rows_check(OutProj& p, size_t n, size_t wo_len, rv_error* err) {
  // prefill.rs:2113-2154 (g): each attention row quantized to Q8_K, the
  // batched o projection, and residual[r][h] += o[h][r] (one f32 add each).
  int32_t rc;
  if ((rc = check_quantize(RV_QF_Q8_K, p.q_dim, p.q_dim / 256, err))) return rc;
  if (!k_quant(p.o_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, p.o_format, 0, 0, "gemv_q8_k_batched");
  return check_gemv("attn_out_proj_rows: weight bytes vs rows / out vs range x n_acts", p.o_format, wo_len, p.q_dim,
                    p.hidden, sat_mul(n, p.q_dim / 256), 0, p.hidden, sat_mul(p.hidden, n), &p.rb, err, n);
}

HipStatus in_proj_rows_launch(const InProj& p, size_t n, hipStream_t s) {
  auto* acts_k = reinterpret_cast<rv_block_q8_k*>(p.scratch);
  auto* acts_0 =
      reinterpret_cast<rv_block_q8_0*>((char*)p.scratch + align16(n * (p.hidden / 256) * sizeof(rv_block_q8_k)));
  // A row of hidden values is a whole number of blocks of both forms, so the
  // rows quantized one after another are one quantization of their concatenation.
  HipStatus st = launch_quantize_both(p.x, acts_k, acts_0, n * (p.hidden / 256), s);
  if (st.e == hipSuccess)
    st = launch_gemv_batched(p.q_format, p.wq, p.rb_q, p.hidden, acts_k, n, 0, p.q_dim, p.q, p.q_dim, true, s);
  if (st.e == hipSuccess)
    st = launch_gemv_batched(RV_QF_Q8_0, p.wk, p.rb_k, p.hidden, acts_0, n, 0, p.kv_dim, p.k, p.kv_dim, true, s);
  if (st.e == hipSuccess)
    st = launch_gemv_batched(p.v_format, p.wv, p.rb_v, p.hidden, acts_k, n, 0, p.kv_dim, p.v, p.kv_dim, true, s);
  return st;
}

HipStatus out_proj_rows_launch(const OutProj& p, size_t n, hipStream_t s) {
  auto* acts = reinterpret_cast<rv_block_q8_k*>(p.scratch);
  HipStatus st = launch_quantize_q8_k(p.x, acts, n * (p.q_dim / 256), s);
  if (st.e == hipSuccess)
    st = launch_gemv_batched(p.o_format, p.wo, p.rb, p.q_dim, acts, n, 0, p.hidden, p.o, p.hidden, true, s, true);
  return st;
}

}  // namespace rv

