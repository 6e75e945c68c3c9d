// rv_block_abi.cpp — one layer's attention block for one token
// (include/ramvamp_block.h; model/forward.rs:2570-2650).
//
// Every check of the five steps runs first, in the reference's order; then
// the input projections (RMSNorm fused), the decode step (prologue, append,
// attention, merge) and the output projection (residual add fused) are
// queued on the cache's stream. `residual` is written only by the last
// launch, so a failure before it leaves the caller's state as it was.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/ramvamp_block.h"
#include "rv_quant.hpp"

namespace {

int32_t fail(rv_error* err, int32_t code, uint64_t a, uint64_t b, const char* what) {
  if (err) *err = rv_error{code, a, b, 0, 0, what};
  return code;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

bool bad_ptr(const void* p) { return !p || ((uintptr_t)p & 3); }

struct Carve {
  float *q, *k, *v, *attn;
  void* proj;
};

Carve carve(void* scratch, size_t q_dim, size_t kv_dim) {
  char* p = (char*)scratch;
  Carve c;
  c.q = (float*)p;
  p += align256(q_dim * sizeof(float));
  c.k = (float*)p;
  p += align256(kv_dim * sizeof(float));
  c.v = (float*)p;
  p += align256(kv_dim * sizeof(float));
  c.attn = (float*)p;
  p += align256(q_dim * sizeof(float));
  c.proj = p;
  return c;
}

}  // namespace

extern "C" {

size_t rv_attn_block_scratch_bytes(size_t hidden, size_t q_dim, size_t kv_dim) {
  const size_t proj = std::max(rv::in_proj_scratch_bytes(hidden, true), rv::out_proj_scratch_bytes(q_dim, hidden, true));
  return 2 * align256(q_dim * sizeof(float)) + 2 * align256(kv_dim * sizeof(float)) + align256(proj);
}

// One token's block at a host position, or (d_position set) at the position
// device memory holds when the step runs, planned for max_position.
static int32_t block_decode(rv_kv* kv, size_t layer, float* residual, size_t hidden, size_t q_dim,
                            const rv_attn_block_weights* w, float eps, float theta, size_t position,
                            const uint32_t* d_position, size_t max_position, float scale, void* scratch,
                            size_t scratch_len, uint32_t flags, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, "kv");
  if (!w) return fail(err, RV_ERR_NULL_ARG, 0, 0, "weights");
  // forward.rs:2572 rmsnorm (norm.rs:38-40): an empty row has no mean.
  if (hidden == 0) return fail(err, RV_PRIM_EMPTY, 0, 0, "rmsnorm");
  const size_t kv_dim = kv->kv_dim;
  const Carve c = carve(scratch, q_dim, kv_dim);
  rv::InProj in{residual, w->attn_norm, eps,     hidden, w->q_format, w->wq, 0,   c.q,   q_dim,
                w->wk,    0,            c.k,     kv_dim, w->v_format, w->wv, 0,   c.v,   c.proj};
  int32_t rc;
  if ((rc = rv::in_proj_check(in, w->wq_len, w->wk_len, w->wv_len, err))) return rc;
  if ((rc = d_position
                ? rv::decode_step_dev_check(kv, layer, q_dim, max_position, w->q_norm_len, w->k_norm_len, err)
                : rv::decode_step_check(kv, layer, q_dim, position, w->q_norm_len, w->k_norm_len, err)))
    return rc;
  rv::OutProj out{c.attn, q_dim, w->o_format, w->wo, 0, residual, hidden, true, c.proj};
  if (d_position) {
    // A refused step (past max_position) leaves the residual as it was.
    out.gate_pos = d_position;
    out.gate_max = (uint32_t)max_position;
  }
  if ((rc = rv::out_proj_check(out, w->wo_len, err))) return rc;
  const size_t need = rv_attn_block_scratch_bytes(hidden, q_dim, kv_dim);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, "attn_block scratch");
  if (flags & RV_HOST_PTRS) return fail(err, RV_ERR_UNSUPPORTED, flags, 0, "RV_HOST_PTRS (device pointers only)");
  const struct {
    const void* p;
    const char* what;
  } ptrs[] = {{residual, "residual"}, {w->attn_norm, "attn_norm"}, {w->wq, "wq"},         {w->wk, "wk"},
              {w->wv, "wv"},          {w->q_norm, "q_norm"},       {w->k_norm, "k_norm"}, {w->wo, "wo"},
              {scratch, "scratch"}};
  for (const auto& p : ptrs)
    if (bad_ptr(p.p)) return fail(err, p.p ? RV_ERR_UNSUPPORTED : RV_ERR_NULL_ARG, (uintptr_t)p.p, 0, p.what);

  int prev = -1;
  if (hipGetDevice(&prev) != hipSuccess) prev = -1;
  if (prev != kv->device) (void)hipSetDevice(kv->device);
  const hipStream_t s = kv->stream;
  rv::HipStatus st = rv::in_proj_launch(in, s);
  if (st.e != hipSuccess) rc = fail(err, RV_ERR_HIP, (uint64_t)st.e, 0, st.what);
  if (!rc && d_position)
    rc = rv_decode_step_dev(kv, layer, c.q, q_dim, c.k, kv_dim, c.v, kv_dim, w->q_norm, w->q_norm_len, w->k_norm,
                            w->k_norm_len, eps, theta, d_position, max_position, scale, c.attn, q_dim, 0, err);
  else if (!rc)
    rc = rv_decode_step(kv, layer, c.q, q_dim, c.k, kv_dim, c.v, kv_dim, w->q_norm, w->q_norm_len, w->k_norm,
                        w->k_norm_len, eps, theta, position, scale, c.attn, q_dim, 0, err);
  if (!rc) {
    st = rv::out_proj_launch(out, s);
    if (st.e != hipSuccess) rc = fail(err, RV_ERR_HIP, (uint64_t)st.e, 0, st.what);
  }
  if (!rc && (flags & RV_SYNC)) {
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = fail(err, RV_ERR_HIP, (uint64_t)e, 0, "hipStreamSynchronize");
  }
  if (prev >= 0 && prev != kv->device) (void)hipSetDevice(prev);
  if (!rc && err) *err = rv_error{RV_OK, 0, 0, 0, 0, nullptr};
  return rc;
}

int32_t rv_attn_block_decode(rv_kv* kv, size_t layer, float* residual, size_t hidden, size_t q_dim,
                             const rv_attn_block_weights* w, float eps, float theta, size_t position,
                             float scale, void* scratch, size_t scratch_len, uint32_t flags, rv_error* err) {
  return block_decode(kv, layer, residual, hidden, q_dim, w, eps, theta, position, nullptr, 0, scale, scratch,
                      scratch_len, flags, err);
}

int32_t rv_attn_block_decode_dev(rv_kv* kv, size_t layer, float* residual, size_t hidden, size_t q_dim,
                                 const rv_attn_block_weights* w, float eps, float theta, const uint32_t* d_position,
                                 size_t max_position, float scale, void* scratch, size_t scratch_len, uint32_t flags,
                                 rv_error* err) {
  if (!d_position) return fail(err, RV_ERR_NULL_ARG, 0, 0, "d_position");
  return block_decode(kv, layer, residual, hidden, q_dim, w, eps, theta, 0, d_position, max_position, scale, scratch,
                      scratch_len, flags, err);
}

// The prefill chunk's scratch: normalized rows, q/k/v rows, attention rows,
// then the projections' quantized rows.
size_t rv_attn_block_prefill_scratch_bytes(size_t n_rows, size_t hidden, size_t q_dim, size_t kv_dim) {
  const size_t proj = std::max(rv::in_proj_rows_scratch_bytes(n_rows, hidden), rv::out_proj_rows_scratch_bytes(n_rows, q_dim));
  return align256(n_rows * hidden * 4) + 2 * align256(n_rows * q_dim * 4) + 2 * align256(n_rows * kv_dim * 4) +
         align256(proj);
}

int32_t rv_attn_block_prefill(rv_kv* kv, size_t layer, float* residual_rows, size_t n_rows, size_t hidden,
                              size_t q_dim, const rv_attn_block_weights* w, float eps, float theta, size_t start,
                              float scale, void* scratch, size_t scratch_len, uint32_t flags, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, "kv");
  if (!w) return fail(err, RV_ERR_NULL_ARG, 0, 0, "weights");
  // prefill.rs:1975-1993 (a): each row's rmsnorm; an empty row has no mean.
  if (hidden == 0) return fail(err, RV_PRIM_EMPTY, 0, 0, "rmsnorm");
  const size_t kv_dim = kv->kv_dim, n = n_rows;
  char* p = (char*)scratch;
  float* normed = (float*)p;
  p += align256(n * hidden * 4);
  float* q = (float*)p;
  p += align256(n * q_dim * 4);
  float* k = (float*)p;
  p += align256(n * kv_dim * 4);
  float* v = (float*)p;
  p += align256(n * kv_dim * 4);
  float* attn = (float*)p;
  p += align256(n * q_dim * 4);
  rv::InProj in{normed, nullptr, 0.f, hidden, w->q_format, w->wq, 0, q, q_dim, w->wk, 0, k, kv_dim,
                w->v_format, w->wv, 0, v, p};
  int32_t rc;
  if ((rc = rv::in_proj_rows_check(in, n, w->wq_len, w->wk_len, w->wv_len, err))) return rc;
  if ((rc = rv::prefill_chunk_check(kv, layer, n, q_dim, start, w->q_norm_len, w->k_norm_len, err))) return rc;
  rv::OutProj out{attn, q_dim, w->o_format, w->wo, 0, residual_rows, hidden, true, p};
  if ((rc = rv::out_proj_rows_check(out, n, w->wo_len, err))) return rc;
  const size_t need = rv_attn_block_prefill_scratch_bytes(n, hidden, q_dim, kv_dim);
  if (scratch_len < need) return fail(err, RV_PRIM_LENGTH_MISMATCH, scratch_len, need, "attn_block_prefill scratch");
  if (flags & RV_HOST_PTRS) return fail(err, RV_ERR_UNSUPPORTED, flags, 0, "RV_HOST_PTRS (device pointers only)");
  if (n == 0) {
    if (err) *err = rv_error{RV_OK, 0, 0, 0, 0, nullptr};
    return RV_OK;
  }
  const struct {
    const void* p;
    const char* what;
  } ptrs[] = {{residual_rows, "residual_rows"}, {w->attn_norm, "attn_norm"}, {w->wq, "wq"},   {w->wk, "wk"},
              {w->wv, "wv"},                    {w->q_norm, "q_norm"},       {w->k_norm, "k_norm"}, {w->wo, "wo"},
              {scratch, "scratch"}};
  for (const auto& ptr : ptrs)
    if (bad_ptr(ptr.p)) return fail(err, ptr.p ? RV_ERR_UNSUPPORTED : RV_ERR_NULL_ARG, (uintptr_t)ptr.p, 0, ptr.what);

  int prev = -1;
  if (hipGetDevice(&prev) != hipSuccess) prev = -1;
  if (prev != kv->device) (void)hipSetDevice(kv->device);
  const hipStream_t s = kv->stream;
  rv::HipStatus st = rv::launch_rmsnorm_rows(residual_rows, w->attn_norm, eps, n, hidden, normed, s);
  if (st.e == hipSuccess) st = rv::in_proj_rows_launch(in, n, s);
  if (st.e != hipSuccess) rc = fail(err, RV_ERR_HIP, (uint64_t)st.e, 0, st.what);
  if (!rc)
    rc = rv_prefill_chunk(kv, layer, q, k, v, n, q_dim, w->q_norm, w->q_norm_len, w->k_norm, w->k_norm_len, eps, theta, start, scale, attn,
                          flags & RV_PREFILL_MODE_MASK, err);
  if (!rc) {
    st = rv::out_proj_rows_launch(out, n, s);
    if (st.e != hipSuccess) rc = fail(err, RV_ERR_HIP, (uint64_t)st.e, 0, st.what);
  }
  if (!rc && (flags & RV_SYNC)) {
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = fail(err, RV_ERR_HIP, (uint64_t)e, 0, "hipStreamSynchronize");
  }
  if (prev >= 0 && prev != kv->device) (void)hipSetDevice(prev);
  if (!rc && err) *err = rv_error{RV_OK, 0, 0, 0, 0, nullptr};
  return rc;
}

}  // extern "C"
