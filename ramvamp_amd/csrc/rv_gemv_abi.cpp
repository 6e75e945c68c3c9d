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

// gemv.rs `validate` (:212-266), n_acts = 1; returns row_bytes.
int32_t check_gemv(const char* what, uint32_t format, size_t weight_len, size_t in_dim, size_t out_dim,
                   size_t act_blocks, size_t row_lo, size_t row_hi, size_t out_len, size_t* row_bytes, rv_error* err) {
  const int32_t rc = rv_quant_row_bytes(format, in_dim, row_bytes, err);
  if (rc) return rc;
  const size_t expected = sat_mul(*row_bytes, out_dim);
  if (expected != weight_len) return fail(err, RV_PRIM_LENGTH_MISMATCH, weight_len, expected, 0, what);
  if (row_lo > row_hi)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, row_lo, row_hi, 0, "gemv rows: row range start vs end");
  if (row_hi > out_dim)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, row_hi, out_dim, 0, "gemv rows: row range end vs out_dim");
  if (out_len != row_hi - row_lo) return fail(err, RV_PRIM_LENGTH_MISMATCH, out_len, row_hi - row_lo, 0, what);
  const size_t wb = in_dim / rv_quant_block_weights(format);
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

size_t rv_attn_in_proj_scratch_bytes(size_t hidden) {
  return align16(hidden / 256 * sizeof(rv_block_q8_k)) + hidden / 32 * sizeof(rv_block_q8_0);
}

int32_t rv_attn_in_proj(const float* normed, size_t hidden, uint32_t q_format, const uint8_t* wq, size_t wq_len,
                        float* q, size_t q_dim, const uint8_t* wk, size_t wk_len, float* k, size_t kv_dim,
                        uint32_t v_format, const uint8_t* wv, size_t wv_len, float* v, void* scratch,
                        size_t scratch_len, void* stream, uint32_t flags, rv_error* err) {
  // forward.rs:2576-2612 in order: both quantizations, then q, k, v.
  int32_t rc;
  if ((rc = check_quantize(RV_QF_Q8_K, hidden, hidden / 256, err))) return rc;
  if ((rc = check_quantize(RV_QF_Q8_0, hidden, hidden / 32, err))) return rc;
  if (!k_quant(q_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, q_format, 0, 0, "attn_in_proj q");
  size_t rb_q, rb_k, rb_v;
  if ((rc = check_gemv("attn_in_proj q: weight bytes vs rows / out vs range", q_format, wq_len, hidden, q_dim,
                       hidden / 256, 0, q_dim, q_dim, &rb_q, err)))
    return rc;
  if ((rc = check_gemv("attn_in_proj k: weight bytes vs rows / out vs range", RV_QF_Q8_0, wk_len, hidden, kv_dim,
                       hidden / 32, 0, kv_dim, kv_dim, &rb_k, err)))
    return rc;
  if (!k_quant(v_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, v_format, 0, 0, "attn_in_proj v");
  if ((rc = check_gemv("attn_in_proj v: weight bytes vs rows / out vs range", v_format, wv_len, hidden, kv_dim,
                       hidden / 256, 0, kv_dim, kv_dim, &rb_v, err)))
    return rc;
  const size_t need = rv_attn_in_proj_scratch_bytes(hidden);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, 0, "attn_in_proj scratch");
  if ((rc = check_flags(flags, err))) return rc;
  if (hidden == 0) return fail(err, RV_ERR_UNSUPPORTED, 0, 0, 0, "attn_in_proj with hidden 0");
  if ((rc = check_ptrs(err, {{normed, "normed"}, {wq, "wq"}, {q, "q"}, {wk, "wk"}, {k, "k"}, {wv, "wv"}, {v, "v"},
                             {scratch, "scratch"}})))
    return rc;
  const hipStream_t s = (hipStream_t)stream;
  if (hidden / 256 <= (size_t)rv::kFusedMaxKBlocks) {
    // One launch: each workgroup quantizes the normed row into LDS (both
    // forms, bit-identical to quantize_row_q8_k / _q8_0) and runs its rows;
    // the quantized row never goes through memory and `scratch` is left
    // untouched.
    rv::FusedProjArgs a{};
    a.x = normed;
    a.nbk = (int)(hidden / 256);
    a.nb0 = (int)(hidden / 32);
    a.n_seg = 3;
    a.seg[0] = {q_format, wq, rb_q, q};
    a.seg[1] = {RV_QF_Q8_0, wk, rb_k, k};
    a.seg[2] = {v_format, wv, rb_v, v};
    a.n_rows[0] = (int)q_dim;
    a.n_rows[1] = (int)kv_dim;
    a.n_rows[2] = (int)kv_dim;
    return finish(s, flags, rv::launch_fused_proj(a, s), err);
  }
  // Wider rows: quantized into `scratch`, then the three GEMVs.
  auto* acts_k = reinterpret_cast<rv_block_q8_k*>(scratch);
  auto* acts_0 = reinterpret_cast<rv_block_q8_0*>((char*)scratch + align16(hidden / 256 * sizeof(rv_block_q8_k)));
  rv::HipStatus st = rv::launch_quantize_q8_k(normed, acts_k, hidden / 256, s);
  if (st.e == hipSuccess) st = rv::launch_quantize_q8_0(normed, acts_0, hidden / 32, s);
  if (st.e == hipSuccess) st = rv::launch_gemv_rows(q_format, wq, rb_q, hidden, acts_k, 0, q_dim, q, s);
  if (st.e == hipSuccess) st = rv::launch_gemv_rows(RV_QF_Q8_0, wk, rb_k, hidden, acts_0, 0, kv_dim, k, s);
  if (st.e == hipSuccess) st = rv::launch_gemv_rows(v_format, wv, rb_v, hidden, acts_k, 0, kv_dim, v, s);
  return finish(s, flags, st, err);
}

size_t rv_attn_out_proj_scratch_bytes(size_t q_dim) { return q_dim / 256 * sizeof(rv_block_q8_k); }

int32_t rv_attn_out_proj(const float* attn_out, size_t q_dim, uint32_t o_format, const uint8_t* wo, size_t wo_len,
                         float* o, size_t hidden, void* scratch, size_t scratch_len, void* stream, uint32_t flags,
                         rv_error* err) {
  // forward.rs:2630-2646: quantize_row_q8_k(attn_out), then the o_proj GEMV.
  int32_t rc;
  if ((rc = check_quantize(RV_QF_Q8_K, q_dim, q_dim / 256, err))) return rc;
  if (!k_quant(o_format)) return fail(err, RV_QUANT_UNSUPPORTED_FORMAT, o_format, 0, 0, "attn_out_proj");
  size_t rb;
  if ((rc = check_gemv("attn_out_proj: weight bytes vs rows / out vs range", o_format, wo_len, q_dim, hidden,
                       q_dim / 256, 0, hidden, hidden, &rb, err)))
    return rc;
  const size_t need = rv_attn_out_proj_scratch_bytes(q_dim);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, 0, "attn_out_proj scratch");
  if ((rc = check_flags(flags, err))) return rc;
  if (q_dim == 0) return fail(err, RV_ERR_UNSUPPORTED, 0, 0, 0, "attn_out_proj with q_dim 0");
  if ((rc = check_ptrs(err, {{attn_out, "attn_out"}, {wo, "wo"}, {o, "o"}, {scratch, "scratch"}}))) return rc;
  const hipStream_t s = (hipStream_t)stream;
  if (q_dim / 256 <= (size_t)rv::kFusedMaxKBlocks) {
    // One launch, the activation quantized into LDS per workgroup (as above).
    rv::FusedProjArgs a{};
    a.x = attn_out;
    a.nbk = (int)(q_dim / 256);
    a.nb0 = (int)(q_dim / 32);
    a.n_seg = 1;
    a.seg[0] = {o_format, wo, rb, o};
    a.n_rows[0] = (int)hidden;
    return finish(s, flags, rv::launch_fused_proj(a, s), err);
  }
  auto* acts = reinterpret_cast<rv_block_q8_k*>(scratch);
  rv::HipStatus st = rv::launch_quantize_q8_k(attn_out, acts, q_dim / 256, s);
  if (st.e == hipSuccess) st = rv::launch_gemv_rows(o_format, wo, rb, q_dim, acts, 0, hidden, o, s);
  return finish(s, flags, st, err);
}

}  // extern "C"
