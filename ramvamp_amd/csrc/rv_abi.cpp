// rv_abi.cpp — the C ABI of include/ramvamp_attn.h.
//
// Host-side validation in the reference's precedence, the per-layer cursors
// of the device KV cache, staging for host pointers, and dispatch to the
// gfx950 kernels (rv_prologue.hip, rv_decode.hip, rv_prefill.hip). Nothing is
// queued on the device before a call's validation has passed, so `out` is
// untouched on every error, as in the reference (attention.rs:413-425).
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <new>

#include "rv_internal.hpp"
#include "../../include/ramvamp_gemv.h"
#include "../../include/ramvamp_router.h"

namespace {

int32_t fail(rv_error* err, int32_t code, uint64_t a = 0, uint64_t b = 0, uint64_t c = 0, uint64_t d = 0,
             const char* what = nullptr) {
  if (err) {
    err->code = code;
    err->a = a;
    err->b = b;
    err->c = c;
    err->d = d;
    err->what = what;
  }
  return code;
}

int32_t ok(rv_error* err) { return fail(err, RV_OK); }

// A HIP failure; a call that would have to allocate under graph capture is
// RV_ERR_UNSUPPORTED instead.
int32_t hip_fail(rv_error* err, hipError_t e, const char* what) {
  return fail(err, rv::status_code(e), (uint64_t)e, 0, 0, 0, what);
}

// Makes the cache's device current for the scope of one call.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

size_t elem_size(int elem) { return elem == RV_ELEM_F32 ? 4 : 2; }

size_t sat_mul(size_t a, size_t b) {
  size_t r;
  return __builtin_mul_overflow(a, b, &r) ? SIZE_MAX : r;
}
size_t sat_add(size_t a, size_t b) {
  size_t r;
  return __builtin_add_overflow(a, b, &r) ? SIZE_MAX : r;
}
size_t scratch_len_of(size_t group, size_t head_dim, size_t max_positions) {
  return sat_add(sat_mul(group, max_positions), sat_mul(head_dim, 2));
}

// kv/mod.rs:190-231 `geometry`.
int32_t geometry(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity, size_t* kv_dim,
                 size_t* plane, size_t* total, rv_error* err) {
  auto invalid = [&](const char* reason) {
    return fail(err, RV_KV_INVALID_DIMS, n_layers, n_kv_heads, head_dim, capacity, reason);
  };
  if (n_layers == 0 || n_kv_heads == 0 || head_dim == 0 || capacity == 0) return invalid("all dims must be nonzero");
  if (__builtin_mul_overflow(n_kv_heads, head_dim, kv_dim)) return invalid("row width overflows usize");
  if (__builtin_mul_overflow(capacity, *kv_dim, plane)) return invalid("plane size overflows usize");
  if (__builtin_mul_overflow(n_layers, *plane, total)) return invalid("total size overflows usize");
  return RV_OK;
}

int32_t check_layer(const rv_kv* kv, size_t layer, rv_error* err) {
  if (layer >= kv->n_layers) return fail(err, RV_KV_LAYER_OUT_OF_RANGE, layer, kv->n_layers);
  return RV_OK;
}

// primitives/norm.rs:72-83 `rmsnorm_in_place` on a head_dim head: q's
// weight first (its heads are normalised first, forward.rs:2622-2627), then
// k's.
int32_t check_norm_weights(size_t hd, size_t q_norm_len, size_t k_norm_len, rv_error* err) {
  if (q_norm_len != hd)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, hd, q_norm_len, 0, 0, "rmsnorm_in_place: x vs weight");
  if (k_norm_len != hd)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, hd, k_norm_len, 0, 0, "rmsnorm_in_place: x vs weight");
  return RV_OK;
}

struct Plan {
  size_t n_q_heads, group, positions;
};

// attention.rs:926-989 `plan`: q length, GQA grouping, layer, positions, kv
// range, out length — the first failure is the one reported.
int32_t plan(const rv_kv* kv, size_t q_len, size_t layer, bool has_limit, size_t limit, size_t kv_lo, size_t kv_hi,
             size_t out_len, Plan* p, rv_error* err) {
  const size_t hd = kv->head_dim, n_kv = kv->n_kv_heads;
  if (q_len == 0 || q_len % hd) return fail(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_len, hd);
  const size_t n_q = q_len / hd;
  if (n_q % n_kv) return fail(err, RV_ATTN_GQA_GROUP_MISMATCH, n_q, n_kv);
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  const size_t len = kv->lens[layer];
  const size_t positions = has_limit ? limit : len;
  if (positions == 0) return fail(err, RV_ATTN_EMPTY_LAYER, layer);
  if (positions > len) return fail(err, RV_KV_POSITION_OUT_OF_RANGE, layer, positions - 1, len);
  if (kv_lo > kv_hi || kv_hi > n_kv) return fail(err, RV_ATTN_KV_HEAD_RANGE, kv_lo, kv_hi, n_kv);
  const size_t group = n_q / n_kv;
  const size_t expected = (kv_hi - kv_lo) * group * hd;
  if (out_len != expected) return fail(err, RV_ATTN_OUT_LEN_MISMATCH, out_len, expected);
  p->n_q_heads = n_q;
  p->group = group;
  p->positions = positions;
  return RV_OK;
}

// Device copies of host-pointer arguments, carved from the cache's staging
// buffer (grown on first need, then reused).
struct Stager {
  rv_kv* kv;
  hipStream_t s;
  size_t used = 0;
  hipError_t e = hipSuccess;
  explicit Stager(rv_kv* k) : kv(k), s(k->stream) {}
  bool reserve(size_t bytes) {
    if (bytes <= kv->stage_bytes) return true;
    if (rv::capturing(s)) {
      e = hipErrorStreamCaptureUnsupported;
      return false;
    }
    void* p = nullptr;
    e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return false;
    if (kv->stage) kv->retire(kv->stage, kv->stage_bytes);
    kv->stage = p;
    kv->stage_bytes = bytes;
    return true;
  }
  static size_t align(size_t n) { return (n + 255) & ~(size_t)255; }
  float* carve(size_t n_floats) {
    float* p = (float*)((char*)kv->stage + used);
    used += align(n_floats * sizeof(float));
    return p;
  }
  float* in(const float* host, size_t n) {
    if (!host || n == 0) return nullptr;
    float* d = carve(n);
    if (e == hipSuccess) e = hipMemcpyAsync(d, host, n * sizeof(float), hipMemcpyHostToDevice, s);
    return d;
  }
};

int32_t finish(rv_kv* kv, uint32_t flags, float* dev_out, float* host_out, size_t n, rv_error* err) {
  if (flags & RV_HOST_PTRS) {
    hipError_t e = hipMemcpyAsync(host_out, dev_out, n * sizeof(float), hipMemcpyDeviceToHost, kv->stream);
    if (e != hipSuccess) return hip_fail(err, e, "hipMemcpyAsync D2H");
    e = hipStreamSynchronize(kv->stream);
    if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  } else if (flags & RV_SYNC) {
    hipError_t e = hipStreamSynchronize(kv->stream);
    if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  }
  return ok(err);
}

// Any attention form after a successful plan.
int32_t run_attention(rv_kv* kv, const float* q, size_t q_len, size_t layer, const Plan& p, float scale, size_t kv_lo,
                      size_t kv_hi, float* out, size_t out_len, uint32_t flags, rv_error* err) {
  if (kv_lo == kv_hi) return ok(err);  // the validated no-op of a surplus shard
  if (!q || !out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !q ? "q" : "out");
  DeviceGuard dg(kv->device);
  const float* dq = q;
  float* dout = out;
  if (flags & RV_HOST_PTRS) {
    Stager st(kv);
    if (!st.reserve(Stager::align(q_len * 4) + Stager::align(out_len * 4))) return hip_fail(err, st.e, "hipMalloc stage");
    dq = st.in(q, q_len);
    dout = st.carve(out_len);
    if (st.e != hipSuccess) return hip_fail(err, st.e, "hipMemcpyAsync H2D");
  }
  rv::HipStatus hs = rv::launch_decode(kv, dq, p.n_q_heads, layer, p.positions, scale, kv_lo, kv_hi, dout, kv->stream);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  return finish(kv, flags, dout, out, out_len, err);
}

int32_t attention_entry(const rv_kv* ckv, const float* q, size_t q_len, size_t layer, bool has_limit, size_t limit,
                        float scale, size_t kv_lo, size_t kv_hi, bool whole, bool check_scratch, size_t scratch_len,
                        float* out, size_t out_len, uint32_t flags, rv_error* err) {
  if (!ckv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  rv_kv* kv = const_cast<rv_kv*>(ckv);
  if (whole) {
    kv_lo = 0;
    kv_hi = kv->n_kv_heads;
  }
  Plan p;
  int32_t rc = plan(kv, q_len, layer, has_limit, limit, kv_lo, kv_hi, out_len, &p, err);
  if (rc) return rc;
  if (check_scratch) {
    const size_t need = scratch_len_of(p.group, kv->head_dim, p.positions);
    if (scratch_len < need) return fail(err, RV_ATTN_SCRATCH_TOO_SHORT, scratch_len, need);
  }
  return run_attention(kv, q, q_len, layer, p, scale, kv_lo, kv_hi, out, out_len, flags, err);
}

// Checks shared by the fused steps: rope needs an even head_dim within the
// inverse-frequency table (primitives/rope.rs:87-88).
int32_t check_rope_dim(const rv_kv* kv, rv_error* err) {
  if (kv->head_dim == 0 || kv->head_dim % 2) return fail(err, RV_PRIM_INVALID_HEAD_DIM, kv->head_dim);
  if (kv->head_dim / 2 > (size_t)rv::kMaxHalf)
    return fail(err, RV_ERR_UNSUPPORTED, kv->head_dim, 0, 0, 0, "head_dim above 512");
  return RV_OK;
}

}  // namespace

namespace rv {

int32_t prefill_chunk_check(const rv_kv* kv, size_t layer, size_t rows, size_t q_dim, size_t start,
                            size_t q_norm_len, size_t k_norm_len, rv_error* err) {
  // rv_prefill_chunk's checks, in its order, before its pointer checks.
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_rope_dim(kv, err);
  if (rc) return rc;
  const size_t hd = kv->head_dim;
  if (q_dim == 0 || q_dim % hd) return fail(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_dim, hd);
  if ((q_dim / hd) % kv->n_kv_heads) return fail(err, RV_ATTN_GQA_GROUP_MISMATCH, q_dim / hd, kv->n_kv_heads);
  if (rows > 0 && (rc = check_norm_weights(hd, q_norm_len, k_norm_len, err))) return rc;
  if ((rc = check_layer(kv, layer, err))) return rc;
  const size_t len = kv->lens[layer];
  if (start != len) return fail(err, RV_KV_POSITION_OUT_OF_RANGE, layer, start, len, 0, "start != len(layer)");
  if (rows > kv->capacity - len) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  if (start + rows > 0x100000000ull) return fail(err, RV_ERR_UNSUPPORTED, start + rows, 0, 0, 0, "position past u32");
  return RV_OK;
}

int32_t decode_step_check(const rv_kv* kv, size_t layer, size_t q_len, size_t position, size_t q_norm_len,
                          size_t k_norm_len, rv_error* err) {
  // rv_decode_step's checks, in its order, for k, v and out of the sizes the
  // cache and q imply (the composite callers own those buffers).
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_rope_dim(kv, err);
  if (rc) return rc;
  const size_t hd = kv->head_dim;
  if (q_len == 0 || q_len % hd) return fail(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_len, hd);
  if ((q_len / hd) % kv->n_kv_heads) return fail(err, RV_ATTN_GQA_GROUP_MISMATCH, q_len / hd, kv->n_kv_heads);
  if ((rc = check_norm_weights(hd, q_norm_len, k_norm_len, err))) return rc;
  if ((rc = check_layer(kv, layer, err))) return rc;
  if (kv->lens[layer] == kv->capacity) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  if (position > 0xFFFFFFFFull) return fail(err, RV_ERR_UNSUPPORTED, position, 0, 0, 0, "position past u32");
  return RV_OK;
}

constexpr size_t kMaxTimedPairs = 4096;  // pairs held before they are folded

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

void timing_fold(rv_kv* kv) {
  for (size_t i = 0; i + 1 < kv->ev_used; i += 2) {
    float ms = 0.f;
    if (hipEventSynchronize(kv->ev[i + 1]) == hipSuccess && hipEventElapsedTime(&ms, kv->ev[i], kv->ev[i + 1]) == hipSuccess) {
      kv->timed_ms += ms;
      kv->timed_n += 1;
    }
  }
  kv->ev_used = 0;
}

TimedPair timing_pair(rv_kv* kv, hipStream_t s) {
  TimedPair tp;
  if (!kv->timing || capturing(s)) return tp;
  if (kv->ev_used + 2 > 2 * kMaxTimedPairs) timing_fold(kv);
  while (kv->ev.size() < kv->ev_used + 2) {
    // Timing-only events: no system-scope fence when they complete, so the
    // timed kernel ends as it would untimed (no extra L2 write-back).
    hipEvent_t e;
    if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return tp;
    kv->ev.push_back(e);
  }
  tp.start = kv->ev[kv->ev_used];
  tp.stop = kv->ev[kv->ev_used + 1];
  kv->ev_used += 2;
  return tp;
}

HipStatus ensure_workspace(rv_kv* kv, size_t bytes, size_t bound) {
  HipStatus st;
  if (bytes <= kv->ws_bytes) return st;
  if (capturing(kv->stream)) {
    st.e = hipErrorStreamCaptureUnsupported;
    st.what = "workspace growth under graph capture (run a call of this shape uncaptured first)";
    return st;
  }
  const size_t want = std::max<size_t>(std::max(bytes, bound), (size_t)1 << 20);
  void* p = nullptr;
  st.e = hipMalloc(&p, want);
  if (st.e != hipSuccess) {
    st.what = "hipMalloc workspace";
    return st;
  }
  if (kv->ws) kv->retire(kv->ws, kv->ws_bytes);
  kv->ws = p;
  kv->ws_bytes = want;
  return st;
}

HipStatus ensure_qbuf(rv_kv* kv, size_t bytes) {
  HipStatus st;
  if (bytes <= kv->qbuf_bytes) return st;
  if (capturing(kv->stream)) {
    st.e = hipErrorStreamCaptureUnsupported;
    st.what = "q buffer growth under graph capture (run a call of this shape uncaptured first)";
    return st;
  }
  void* p = nullptr;
  st.e = hipMalloc(&p, bytes);
  if (st.e != hipSuccess) {
    st.what = "hipMalloc qbuf";
    return st;
  }
  if (kv->qbuf) kv->retire(kv->qbuf, kv->qbuf_bytes);
  kv->qbuf = (float*)p;
  kv->qbuf_bytes = bytes;
  return st;
}

// The device-position step's (cos, sin) table for positions [0, n) at
// theta: each position's 64 pairs in f64 from the host's inverse
// frequencies, cast to f32, exactly as rv_decode_step computes its one
// position's (rope.rs:35-39), for whole blocks of 1024 positions up to the
// capacity; extended (or rebuilt for another theta) on need, the replaced
// table retired rather than freed.
HipStatus ensure_rope_tab(rv_kv* kv, float theta, size_t n) {
  HipStatus st;
  if (kv->rope_tab && kv->rope_theta == theta && kv->rope_n >= n) return st;
  if (capturing(kv->stream)) {
    st.e = hipErrorStreamCaptureUnsupported;
    st.what = "rope table growth under graph capture (run a device-position step uncaptured first)";
    return st;
  }
  const size_t hd = kv->head_dim, half = hd / 2;
  const size_t rows = std::min(kv->capacity, (n + 1023) / 1024 * 1024);
  std::vector<float> host(rows * hd);
  InvFreq inv;
  fill_inv_freq(inv, hd, theta);
  for (size_t p = 0; p < rows; ++p)
    for (size_t i = 0; i < half; ++i) {
      double sd, cd;
      sincos((double)p * inv.f[i], &sd, &cd);
      host[p * hd + i] = (float)cd;
      host[p * hd + half + i] = (float)sd;
    }
  void* d = nullptr;
  st.e = hipMalloc(&d, host.size() * sizeof(float));
  if (st.e != hipSuccess) {
    st.what = "hipMalloc rope table";
    return st;
  }
  st.e = hipMemcpy(d, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice);
  if (st.e != hipSuccess) {
    (void)hipFree(d);
    st.what = "hipMemcpy rope table";
    return st;
  }
  if (kv->rope_tab) kv->retire(kv->rope_tab, kv->rope_n * kv->head_dim * sizeof(float));
  kv->rope_tab = (float*)d;
  kv->rope_n = rows;
  kv->rope_theta = theta;
  return st;
}

int32_t decode_step_dev_check(const rv_kv* kv, size_t layer, size_t q_len, size_t max_position, size_t q_norm_len,
                              size_t k_norm_len, rv_error* err) {
  // rv_decode_step's checks with the token's position on the device: the
  // launch is planned for max_position, which must leave a row for it.
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_rope_dim(kv, err);
  if (rc) return rc;
  const size_t hd = kv->head_dim;
  if (q_len == 0 || q_len % hd) return fail(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_len, hd);
  if ((q_len / hd) % kv->n_kv_heads) return fail(err, RV_ATTN_GQA_GROUP_MISMATCH, q_len / hd, kv->n_kv_heads);
  if ((rc = check_norm_weights(hd, q_norm_len, k_norm_len, err))) return rc;
  if ((rc = check_layer(kv, layer, err))) return rc;
  if (max_position >= kv->capacity) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  if (!decode_pro_supported(kv, q_len / hd))
    return fail(err, RV_ERR_UNSUPPORTED, hd, q_len / hd / kv->n_kv_heads, 0, 0,
                "device-position step: head_dim 128 and a group of at most 16");
  return RV_OK;
}

}  // namespace rv

extern "C" {

uint32_t rv_abi_version(void) { return RV_ABI_VERSION; }

const char* rv_status_name(int32_t code) {
  switch (code) {
    case RV_OK: return "RV_OK";
    case RV_KV_INVALID_DIMS: return "RV_KV_INVALID_DIMS";
    case RV_KV_LAYER_OUT_OF_RANGE: return "RV_KV_LAYER_OUT_OF_RANGE";
    case RV_KV_ROW_LEN_MISMATCH: return "RV_KV_ROW_LEN_MISMATCH";
    case RV_KV_CAPACITY_EXCEEDED: return "RV_KV_CAPACITY_EXCEEDED";
    case RV_KV_POSITION_OUT_OF_RANGE: return "RV_KV_POSITION_OUT_OF_RANGE";
    case RV_KV_RAGGED_LAYERS: return "RV_KV_RAGGED_LAYERS";
    case RV_KV_TRUNCATE_BEYOND_LENGTH: return "RV_KV_TRUNCATE_BEYOND_LENGTH";
    case RV_ATTN_Q_LEN_INDIVISIBLE: return "RV_ATTN_Q_LEN_INDIVISIBLE";
    case RV_ATTN_GQA_GROUP_MISMATCH: return "RV_ATTN_GQA_GROUP_MISMATCH";
    case RV_ATTN_OUT_LEN_MISMATCH: return "RV_ATTN_OUT_LEN_MISMATCH";
    case RV_ATTN_EMPTY_LAYER: return "RV_ATTN_EMPTY_LAYER";
    case RV_ATTN_KV_HEAD_RANGE: return "RV_ATTN_KV_HEAD_RANGE";
    case RV_ATTN_SCRATCH_TOO_SHORT: return "RV_ATTN_SCRATCH_TOO_SHORT";
    case RV_PRIM_INVALID_HEAD_DIM: return "RV_PRIM_INVALID_HEAD_DIM";
    case RV_PRIM_LENGTH_MISMATCH: return "RV_PRIM_LENGTH_MISMATCH";
    case RV_PRIM_EMPTY: return "RV_PRIM_EMPTY";
    case RV_FWD_INVALID_TOP_K: return "RV_FWD_INVALID_TOP_K";
    case RV_ERR_NULL_ARG: return "RV_ERR_NULL_ARG";
    case RV_ERR_UNSUPPORTED: return "RV_ERR_UNSUPPORTED";
    case RV_ERR_HIP: return "RV_ERR_HIP";
    case RV_ERR_BAD_ELEM: return "RV_ERR_BAD_ELEM";
    case RV_QUANT_INDIVISIBLE_ROW: return "RV_QUANT_INDIVISIBLE_ROW";
    case RV_QUANT_ROW_BYTES_NOT_BLOCK_MULTIPLE: return "RV_QUANT_ROW_BYTES_NOT_BLOCK_MULTIPLE";
    case RV_QUANT_BLOCK_COUNT_MISMATCH: return "RV_QUANT_BLOCK_COUNT_MISMATCH";
    case RV_QUANT_QUANTIZE_LEN_MISMATCH: return "RV_QUANT_QUANTIZE_LEN_MISMATCH";
    case RV_QUANT_UNSUPPORTED_FORMAT: return "RV_QUANT_UNSUPPORTED_FORMAT";
    default: return "RV_UNKNOWN";
  }
}

size_t rv_scratch_len(size_t n_q_heads, size_t n_kv_heads, size_t head_dim, size_t max_positions) {
  const size_t group = n_kv_heads ? n_q_heads / n_kv_heads : 0;
  return scratch_len_of(group, head_dim, max_positions);
}

int32_t rv_kv_projected_bytes(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity, rv_elem elem,
                              uint64_t* bytes, rv_error* err) {
  if (elem != RV_ELEM_F16 && elem != RV_ELEM_F32) return fail(err, RV_ERR_BAD_ELEM, (uint64_t)elem);
  if (!bytes) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "bytes");
  size_t kv_dim, plane, total, b2, b;
  int32_t rc = geometry(n_layers, n_kv_heads, head_dim, capacity, &kv_dim, &plane, &total, err);
  if (rc) return rc;
  if (__builtin_mul_overflow(total, (size_t)2, &b2) || __builtin_mul_overflow(b2, elem_size(elem), &b))
    return fail(err, RV_KV_INVALID_DIMS, n_layers, n_kv_heads, head_dim, capacity,
                "total size in bytes overflows usize");
  *bytes = (uint64_t)b;
  return ok(err);
}

int32_t rv_kv_new(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity, rv_elem elem, int device,
                  rv_kv** out, rv_error* err) {
  if (!out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "out");
  uint64_t bytes;
  int32_t rc = rv_kv_projected_bytes(n_layers, n_kv_heads, head_dim, capacity, elem, &bytes, err);
  if (rc) return rc;
  rv_kv* kv = new (std::nothrow) rv_kv();
  if (!kv) return fail(err, RV_ERR_HIP, (uint64_t)hipErrorOutOfMemory, 0, 0, 0, "host allocation");
  size_t total;
  geometry(n_layers, n_kv_heads, head_dim, capacity, &kv->kv_dim, &kv->plane, &total, nullptr);
  kv->n_layers = n_layers;
  kv->n_kv_heads = n_kv_heads;
  kv->head_dim = head_dim;
  kv->capacity = capacity;
  kv->elem = elem;
  kv->device = device;
  kv->lens.assign(n_layers, 0);
  kv->staged.assign(n_layers, nullptr);
  kv->staged_bytes.assign(n_layers, 0);
  kv->staged_pos.assign(n_layers, 0);
  kv->staged_mode.assign(n_layers, 0);
  DeviceGuard dg(device);
  const size_t plane_bytes = total * elem_size(elem);
  hipError_t e = hipMalloc(&kv->k, plane_bytes);
  if (e == hipSuccess) e = hipMalloc(&kv->v, plane_bytes);
  if (e == hipSuccess) e = hipMemset(kv->k, 0, plane_bytes);
  if (e == hipSuccess) e = hipMemset(kv->v, 0, plane_bytes);
  const size_t ticket_bytes = rv::ticket_words(kv) * sizeof(unsigned);
  if (e == hipSuccess) e = hipMalloc(&kv->tickets, ticket_bytes);
  if (e == hipSuccess) e = hipMemset(kv->tickets, 0, ticket_bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) kv->xcd_ok = rv::xcd_dealing_ok(device);
  if (e == hipSuccess) {
    const rv::HipStatus st = rv::ensure_workspace(kv, rv::decode_ws_bound(kv));
    e = st.e;
  }
  if (e == hipSuccess) {
    // Set-up of rv_decode_attention_noalloc on this device (its scratch
    // array's address), so that its calls never resolve it themselves.
    void* scratch = nullptr;
    (void)rv::noalloc_scratch(device, &scratch);
  }
  if (e != hipSuccess) {
    rv_kv_free(kv);
    return hip_fail(err, e, "hipMalloc planes");
  }
  *out = kv;
  return ok(err);
}

void rv_kv_free(rv_kv* kv) {
  if (!kv) return;
  {
    DeviceGuard dg(kv->device);
    if (kv->stream) (void)hipStreamSynchronize(kv->stream);
    else (void)hipDeviceSynchronize();
    for (void* p : {kv->k, kv->v, kv->ws, (void*)kv->qbuf, kv->stage, (void*)kv->tickets, (void*)kv->rope_tab,
                    (void*)kv->pf_tickets})
      if (p) (void)hipFree(p);
    for (void* p : kv->staged)
      if (p) (void)hipFree(p);
    for (void* p : kv->retired) (void)hipFree(p);
    for (hipEvent_t e : kv->ev) (void)hipEventDestroy(e);
    if (kv->order_ev) (void)hipEventDestroy(kv->order_ev);
  }
  delete kv;
}

// The cache's planes, workspace and staged copies are shared by every call,
// so work queued on the new stream is ordered after what the old one holds.
// Not across a graph capture: an event recorded outside a capture cannot
// order work inside it (a capture's work runs when the graph is launched).
int32_t rv_kv_set_stream(rv_kv* kv, void* hip_stream, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  const hipStream_t next = (hipStream_t)hip_stream;
  if (next == kv->stream) return ok(err);
  DeviceGuard dg(kv->device);
  if (rv::capturing(next) || rv::capturing(kv->stream)) {
    kv->stream = next;
    return ok(err);
  }
  if (!kv->order_ev) {
    const hipError_t e = hipEventCreateWithFlags(&kv->order_ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      kv->order_ev = nullptr;
      return hip_fail(err, e, "hipEventCreate (stream hand-over)");
    }
  }
  hipError_t e = hipEventRecord(kv->order_ev, kv->stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(next, kv->order_ev, 0);
  if (e != hipSuccess) return hip_fail(err, e, "stream hand-over");
  kv->stream = next;
  return ok(err);
}

int32_t rv_kv_synchronize(rv_kv* kv, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  DeviceGuard dg(kv->device);
  hipError_t e = hipStreamSynchronize(kv->stream);
  if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  return ok(err);
}

size_t rv_kv_n_layers(const rv_kv* kv) { return kv ? kv->n_layers : 0; }
size_t rv_kv_n_kv_heads(const rv_kv* kv) { return kv ? kv->n_kv_heads : 0; }
size_t rv_kv_head_dim(const rv_kv* kv) { return kv ? kv->head_dim : 0; }
size_t rv_kv_capacity(const rv_kv* kv) { return kv ? kv->capacity : 0; }
size_t rv_kv_kv_dim(const rv_kv* kv) { return kv ? kv->kv_dim : 0; }
int32_t rv_kv_elem(const rv_kv* kv) { return kv ? kv->elem : 0; }

int32_t rv_kv_len(const rv_kv* kv, size_t layer, size_t* len, rv_error* err) {
  if (!kv || !len) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !kv ? "kv" : "len");
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  *len = kv->lens[layer];
  return ok(err);
}

int rv_kv_is_empty(const rv_kv* kv) {
  if (!kv) return 1;
  for (size_t l : kv->lens)
    if (l) return 0;
  return 1;
}

// kv/mod.rs:312-325.
int32_t rv_kv_seq_len(const rv_kv* kv, size_t* len, rv_error* err) {
  if (!kv || !len) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !kv ? "kv" : "len");
  const auto mm = std::minmax_element(kv->lens.begin(), kv->lens.end());
  if (*mm.first != *mm.second) return fail(err, RV_KV_RAGGED_LAYERS, *mm.first, *mm.second);
  *len = *mm.first;
  return ok(err);
}

int32_t rv_kv_append_rows(rv_kv* kv, size_t layer, const float* k, const float* v, size_t rows, size_t row_len,
                          uint32_t flags, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  if (row_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, row_len, kv->kv_dim, 0, 0, "k");
  const size_t len = kv->lens[layer];
  if (rows > kv->capacity - len) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  if (rows == 0) return ok(err);
  if (!k || !v) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !k ? "k" : "v");
  DeviceGuard dg(kv->device);
  const float* dk = k;
  const float* dv = v;
  if (flags & RV_HOST_PTRS) {
    Stager st(kv);
    const size_t n = rows * kv->kv_dim;
    if (!st.reserve(2 * Stager::align(n * 4))) return hip_fail(err, st.e, "hipMalloc stage");
    dk = st.in(k, n);
    dv = st.in(v, n);
    if (st.e != hipSuccess) return hip_fail(err, st.e, "hipMemcpyAsync H2D");
  }
  rv::HipStatus hs = rv::launch_append(kv, layer, len, dk, dv, rows, kv->stream);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  kv->lens[layer] = len + rows;
  if (flags & (RV_HOST_PTRS | RV_SYNC)) {
    hipError_t e = hipStreamSynchronize(kv->stream);
    if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  }
  return ok(err);
}

// kv/mod.rs:336-368: layer, k length, v length, capacity.
int32_t rv_kv_append(rv_kv* kv, size_t layer, const float* k, size_t k_len, const float* v, size_t v_len,
                     uint32_t flags, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  if (k_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, k_len, kv->kv_dim, 0, 0, "k");
  if (v_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, v_len, kv->kv_dim, 0, 0, "v");
  if (kv->lens[layer] == kv->capacity) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  return rv_kv_append_rows(kv, layer, k, v, 1, kv->kv_dim, flags, err);
}

void rv_kv_clear(rv_kv* kv) {
  if (!kv) return;
  std::fill(kv->lens.begin(), kv->lens.end(), 0);
  std::fill(kv->staged_pos.begin(), kv->staged_pos.end(), 0);
}

// kv/mod.rs:410-420: ragged first, then an upward target.
int32_t rv_kv_truncate(rv_kv* kv, size_t new_len, rv_error* err) {
  size_t len;
  int32_t rc = rv_kv_seq_len(kv, &len, err);
  if (rc) return rc;
  if (new_len > len) return fail(err, RV_KV_TRUNCATE_BEYOND_LENGTH, new_len, len);
  std::fill(kv->lens.begin(), kv->lens.end(), new_len);
  // Rows from new_len on will be rewritten: their staged copies are stale.
  for (size_t& sp : kv->staged_pos) sp = std::min(sp, new_len);
  return ok(err);
}

static int32_t layer_view(const rv_kv* kv, int plane_v, size_t layer, const void** dev, size_t* n, rv_error* err) {
  if (!kv || !dev || !n) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv/dev/n_elems");
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  *dev = plane_v ? kv->v_layer(layer) : kv->k_layer(layer);
  *n = kv->lens[layer] * kv->kv_dim;
  return ok(err);
}

int32_t rv_kv_k_layer(const rv_kv* kv, size_t layer, const void** dev, size_t* n_elems, rv_error* err) {
  return layer_view(kv, 0, layer, dev, n_elems, err);
}
int32_t rv_kv_v_layer(const rv_kv* kv, size_t layer, const void** dev, size_t* n_elems, rv_error* err) {
  return layer_view(kv, 1, layer, dev, n_elems, err);
}

int32_t rv_kv_read_row(const rv_kv* kv, int plane_v, size_t layer, size_t pos, void* dst, rv_error* err) {
  if (!kv || !dst) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !kv ? "kv" : "dst");
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  const size_t len = kv->lens[layer];
  if (pos >= len) return fail(err, RV_KV_POSITION_OUT_OF_RANGE, layer, pos, len);
  DeviceGuard dg(kv->device);
  const size_t es = kv->elem_size();
  const char* src = (plane_v ? kv->v_layer(layer) : kv->k_layer(layer)) + pos * kv->kv_dim * es;
  hipError_t e = hipMemcpyAsync(dst, src, kv->kv_dim * es, hipMemcpyDeviceToHost, kv->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(kv->stream);
  if (e != hipSuccess) return hip_fail(err, e, "read_row");
  return ok(err);
}

int32_t rv_decode_attention(const rv_kv* kv, const float* q, size_t q_len, size_t layer, float scale, float* out,
                            size_t out_len, uint32_t flags, rv_error* err) {
  return attention_entry(kv, q, q_len, layer, false, 0, scale, 0, 0, true, false, 0, out, out_len, flags, err);
}

// No reference counterpart: rv_decode_attention on the device scratch array
// (rv_decode.hip), allocating nothing.
int32_t rv_decode_attention_noalloc(const rv_kv* ckv, const float* q, size_t q_len, size_t layer, float scale,
                                    float* out, size_t out_len, uint32_t flags, rv_error* err) {
  if (!ckv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  rv_kv* kv = const_cast<rv_kv*>(ckv);
  if (flags & RV_HOST_PTRS)
    return fail(err, RV_ERR_UNSUPPORTED, 0, rv::kNoAllocScratchBytes, 0, 0, "host pointers (staging allocates)");
  Plan p;
  int32_t rc = plan(kv, q_len, layer, false, 0, 0, kv->n_kv_heads, out_len, &p, err);
  if (rc) return rc;
  if (!q || !out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !q ? "q" : "out");
  const size_t need = rv::decode_ws_need(kv, p.n_q_heads, p.positions, kv->n_kv_heads);
  if (need > rv::kNoAllocScratchBytes)
    return fail(err, RV_ERR_UNSUPPORTED, need, rv::kNoAllocScratchBytes, 0, 0, "decode scratch above the no-alloc limit");
  DeviceGuard dg(kv->device);
  void* base = nullptr;
  rv::HipStatus hs = rv::noalloc_scratch(kv->device, &base);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  const rv::Workspace ws{base, rv::kNoAllocScratchBytes};
  hs = rv::launch_decode(kv, q, p.n_q_heads, layer, p.positions, scale, 0, kv->n_kv_heads, out, kv->stream, &ws);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  if (flags & RV_SYNC) {
    const hipError_t e = hipStreamSynchronize(kv->stream);
    if (e != hipSuccess) return hip_fail(err, e, "hipStreamSynchronize");
  }
  return ok(err);
}

int32_t rv_decode_attention_in(const rv_kv* kv, const float* q, size_t q_len, size_t layer, float scale,
                               size_t scratch_len, float* out, size_t out_len, uint32_t flags, rv_error* err) {
  return attention_entry(kv, q, q_len, layer, false, 0, scale, 0, 0, true, true, scratch_len, out, out_len, flags,
                         err);
}

int32_t rv_decode_attention_kv_range_in(const rv_kv* kv, const float* q, size_t q_len, size_t layer, float scale,
                                        size_t kv_lo, size_t kv_hi, size_t scratch_len, float* out, size_t out_len,
                                        uint32_t flags, rv_error* err) {
  return attention_entry(kv, q, q_len, layer, false, 0, scale, kv_lo, kv_hi, false, true, scratch_len, out, out_len,
                         flags, err);
}

int32_t rv_attention_at(const rv_kv* kv, const float* q, size_t q_len, size_t layer, size_t positions, float scale,
                        float* out, size_t out_len, uint32_t flags, rv_error* err) {
  return attention_entry(kv, q, q_len, layer, true, positions, scale, 0, 0, true, false, 0, out, out_len, flags, err);
}

int32_t rv_attention_at_in(const rv_kv* kv, const float* q, size_t q_len, size_t layer, size_t positions, float scale,
                           size_t scratch_len, float* out, size_t out_len, uint32_t flags, rv_error* err) {
  return attention_entry(kv, q, q_len, layer, true, positions, scale, 0, 0, true, true, scratch_len, out, out_len,
                         flags, err);
}

int32_t rv_attention_at_kv_range_in(const rv_kv* kv, const float* q, size_t q_len, size_t layer, size_t positions,
                                    float scale, size_t kv_lo, size_t kv_hi, size_t scratch_len, float* out,
                                    size_t out_len, uint32_t flags, rv_error* err) {
  return attention_entry(kv, q, q_len, layer, true, positions, scale, kv_lo, kv_hi, false, true, scratch_len, out,
                         out_len, flags, err);
}

// Row-batched causal attention, validated row by row in order before launch.
static int32_t rows_plan(const rv_kv* kv, size_t rows, size_t q_dim, size_t layer, size_t start, Plan* p,
                         rv_error* err) {
  // Row 0 carries every check but the position limit's growth; the first row
  // whose limit passes the layer length is the first failure after it.
  int32_t rc = plan(kv, q_dim, layer, true, start + 1, 0, kv->n_kv_heads, q_dim, p, err);
  if (rc) return rc;
  const size_t len = kv->lens[layer];
  if (start + rows > len) {
    const size_t r = len - start;  // first row with start + r + 1 > len
    return fail(err, RV_KV_POSITION_OUT_OF_RANGE, layer, start + r, len);
  }
  return RV_OK;
}

static int32_t run_rows(rv_kv* kv, const float* dq, size_t rows, size_t q_dim, size_t layer, size_t start,
                        const Plan& p, float scale, float* dout, uint32_t flags, rv_error* err) {
  rv::HipStatus hs;
  if (rv::prefill_supported(kv, p.group, start + rows)) {
    hs = rv::launch_prefill(kv, dq, rows, p.n_q_heads, layer, start, scale, dout, flags, nullptr, kv->stream);
  } else {
    for (size_t r = 0; r < rows && hs.e == hipSuccess; ++r)
      hs = rv::launch_decode(kv, dq + r * q_dim, p.n_q_heads, layer, start + r + 1, scale, 0, kv->n_kv_heads,
                             dout + r * q_dim, kv->stream);
  }
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  return RV_OK;
}

int32_t rv_attention_at_rows(const rv_kv* ckv, const float* q_rows, size_t rows, size_t q_dim, size_t layer,
                             size_t start, float scale, float* out, uint32_t flags, rv_error* err) {
  if (!ckv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  rv_kv* kv = const_cast<rv_kv*>(ckv);
  if (rows == 0) return ok(err);  // prefill.rs:1335-1337
  Plan p;
  int32_t rc = rows_plan(kv, rows, q_dim, layer, start, &p, err);
  if (rc) return rc;
  if (!q_rows || !out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !q_rows ? "q_rows" : "out");
  DeviceGuard dg(kv->device);
  const size_t n = rows * q_dim;
  const float* dq = q_rows;
  float* dout = out;
  if (flags & RV_HOST_PTRS) {
    Stager st(kv);
    if (!st.reserve(2 * Stager::align(n * 4))) return hip_fail(err, st.e, "hipMalloc stage");
    dq = st.in(q_rows, n);
    dout = st.carve(n);
    if (st.e != hipSuccess) return hip_fail(err, st.e, "hipMemcpyAsync H2D");
  }
  rc = run_rows(kv, dq, rows, q_dim, layer, start, p, scale, dout, flags, err);
  if (rc) return rc;
  return finish(kv, flags, dout, out, n, err);
}

// model/forward.rs:2622-2633.
int32_t rv_decode_step(rv_kv* kv, size_t layer, const float* q, size_t q_len, const float* k, size_t k_len,
                       const float* v, size_t v_len, const float* q_norm_w, size_t q_norm_len,
                       const float* k_norm_w, size_t k_norm_len, float eps, float theta, size_t position,
                       float scale, float* out, size_t out_len, uint32_t flags, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_rope_dim(kv, err);
  if (rc) return rc;
  const size_t hd = kv->head_dim;
  if (q_len == 0 || q_len % hd) return fail(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_len, hd);
  if ((q_len / hd) % kv->n_kv_heads) return fail(err, RV_ATTN_GQA_GROUP_MISMATCH, q_len / hd, kv->n_kv_heads);
  if ((rc = check_norm_weights(hd, q_norm_len, k_norm_len, err))) return rc;
  if ((rc = check_layer(kv, layer, err))) return rc;
  if (k_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, k_len, kv->kv_dim, 0, 0, "k");
  if (v_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, v_len, kv->kv_dim, 0, 0, "v");
  const size_t len = kv->lens[layer];
  if (len == kv->capacity) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  if (out_len != q_len) return fail(err, RV_ATTN_OUT_LEN_MISMATCH, out_len, q_len);
  if (position > 0xFFFFFFFFull) return fail(err, RV_ERR_UNSUPPORTED, position, 0, 0, 0, "position past u32");
  if (!q || !k || !v || !q_norm_w || !k_norm_w || !out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "tensor");
  DeviceGuard dg(kv->device);
  const float *dq = q, *dk = k, *dv = v, *dwq = q_norm_w, *dwk = k_norm_w;
  float* dout = out;
  if (flags & RV_HOST_PTRS) {
    Stager st(kv);
    const size_t need = 2 * Stager::align(q_len * 4) + 2 * Stager::align(kv->kv_dim * 4) + 2 * Stager::align(hd * 4);
    if (!st.reserve(need)) return hip_fail(err, st.e, "hipMalloc stage");
    dq = st.in(q, q_len);
    dk = st.in(k, kv->kv_dim);
    dv = st.in(v, kv->kv_dim);
    dwq = st.in(q_norm_w, hd);
    dwk = st.in(k_norm_w, hd);
    dout = st.carve(q_len);
    if (st.e != hipSuccess) return hip_fail(err, st.e, "hipMemcpyAsync H2D");
  }
  rv::InvFreq inv;
  rv::fill_inv_freq(inv, hd, theta);
  const size_t n_q = q_len / hd;
  if (rv::decode_pro_supported(kv, n_q)) {
    // One launch (plus the split merge): the prologue runs in the tile
    // kernel; (cos, sin) of the position in f64, as rope.rs:35-39.
    rv::DecodePro pro{dk, dv, dwq, dwk, eps, {}, {}};
    const double pos = (double)position;
    for (size_t i = 0; i < hd / 2; ++i) {
      double sd, cd;
      sincos(pos * inv.f[i], &sd, &cd);
      pro.cs[i] = (float)cd;
      pro.sn[i] = (float)sd;
    }
    kv->lens[layer] = len + 1;
    rv::HipStatus hs = rv::launch_decode_pro(kv, dq, n_q, layer, len + 1, scale, pro, dout, kv->stream);
    if (hs.e != hipSuccess) {
      kv->lens[layer] = len;
      return hip_fail(err, hs.e, hs.what);
    }
    return finish(kv, flags, dout, out, q_len, err);
  }
  rv::HipStatus hs = rv::ensure_qbuf(kv, q_len * sizeof(float));
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  // q and k rotate at `position` (forward.rs:2628-2629); the row lands at
  // the layer's cursor.
  hs = rv::launch_row_prologue(kv, layer, len, dq, kv->qbuf, n_q, dk, dv, 1, dwq, dwk, eps, inv, position, nullptr,
                               nullptr, kv->stream);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  kv->lens[layer] = len + 1;
  hs = rv::launch_decode(kv, kv->qbuf, n_q, layer, len + 1, scale, 0, kv->n_kv_heads, dout, kv->stream);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  return finish(kv, flags, dout, out, q_len, err);
}

// rv_decode_step with the token's position read from device memory when the
// step runs, for a token graph captured once and replayed for every token.
int32_t rv_decode_step_dev(rv_kv* kv, size_t layer, const float* q, size_t q_len, const float* k, size_t k_len,
                           const float* v, size_t v_len, const float* q_norm_w, size_t q_norm_len,
                           const float* k_norm_w, size_t k_norm_len, float eps, float theta,
                           const uint32_t* d_position, size_t max_position, float scale, float* out, size_t out_len,
                           uint32_t flags, rv_error* err) {
  int32_t rc = rv::decode_step_dev_check(kv, layer, q_len, max_position, q_norm_len, k_norm_len, err);
  if (rc) return rc;
  if (k_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, k_len, kv->kv_dim, 0, 0, "k");
  if (v_len != kv->kv_dim) return fail(err, RV_KV_ROW_LEN_MISMATCH, v_len, kv->kv_dim, 0, 0, "v");
  if (out_len != q_len) return fail(err, RV_ATTN_OUT_LEN_MISMATCH, out_len, q_len);
  if (!q || !k || !v || !q_norm_w || !k_norm_w || !out || !d_position)
    return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "tensor");
  if (flags & RV_HOST_PTRS) return fail(err, RV_ERR_UNSUPPORTED, flags, 0, 0, 0, "RV_HOST_PTRS (device pointers only)");
  DeviceGuard dg(kv->device);
  rv::HipStatus hs = rv::ensure_rope_tab(kv, theta, max_position + 1);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  rv::DecodePro pro{k, v, q_norm_w, k_norm_w, eps, {}, {}, d_position, kv->rope_tab, (int)max_position,
                    rv::dev_status(kv), (uint32_t)layer};
  hs = rv::launch_decode_pro(kv, q, q_len / kv->head_dim, layer, max_position + 1, scale, pro, out, kv->stream);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  return finish(kv, flags, out, out, q_len, err);
}

// Rows that device-position steps wrote below the layer's capacity, added to
// its host cursor (kv/mod.rs:336-368's bound).
int32_t rv_kv_commit(rv_kv* kv, size_t layer, size_t rows, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  if ((rc = rv_kv_device_status(kv, err))) return rc;
  if (rows > kv->capacity - kv->lens[layer]) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  kv->lens[layer] += rows;
  return ok(err);
}

// The status word a device-position step leaves when it refuses a position
// past its plan (rv_decode.hip): [0] code, [1] layer, [2] position read,
// [3] the step's max_position + 1. Read after the stream drains, then cleared.
int32_t rv_kv_device_status(rv_kv* kv, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  DeviceGuard dg(kv->device);
  uint32_t w[4] = {0, 0, 0, 0};
  hipError_t e = kv->stream ? hipStreamSynchronize(kv->stream) : hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(w, rv::dev_status(kv), sizeof(w), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(err, e, "read the device status");
  if (w[0] == 0) return ok(err);
  const uint32_t zero[4] = {0, 0, 0, 0};
  e = hipMemcpy(rv::dev_status(kv), zero, sizeof(zero), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(err, e, "clear the device status");
  return fail(err, (int32_t)w[0], w[1], w[3], w[2], 0, "device-position step past its planned positions");
}

int32_t rv_kv_device_bytes(rv_kv* kv, uint64_t* now, uint64_t* bound, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  const size_t planes = 2 * kv->n_layers * kv->plane * kv->elem_size();
  size_t staged = 0;
  for (size_t b : kv->staged_bytes) staged += b;
  const size_t base = planes + kv->ws_bytes + kv->qbuf_bytes + kv->stage_bytes + kv->retired_bytes +
                      rv::ticket_words(kv) * sizeof(unsigned);
  const size_t tab = kv->rope_n * kv->head_dim * sizeof(float);
  if (now) *now = (uint64_t)(base + tab + staged);
  if (bound) {
    // Every layer's staged copy at its capacity in the costliest mode, the
    // table over the whole capacity; a copy already made in another mode
    // was retired (counted in base) when it was replaced.
    const size_t per_layer = rv::prefill_stage_bound(kv);
    size_t st = 0;
    for (size_t b : kv->staged_bytes) st += std::max(b, per_layer);
    const size_t tab_cap = std::max(tab, kv->capacity * kv->head_dim * sizeof(float));
    *bound = (uint64_t)(base + tab_cap + st);
  }
  return ok(err);
}

int32_t rv_kv_projected_device_bytes(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity,
                                     rv_elem elem, uint64_t* bytes, rv_error* err) {
  uint64_t planes = 0;
  int32_t rc = rv_kv_projected_bytes(n_layers, n_kv_heads, head_dim, capacity, elem, &planes, err);
  if (rc) return rc;
  if (!bytes) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "bytes");
  // The host fields the sizing reads, as rv_kv_new sets them (no device
  // memory is touched).
  rv_kv g;
  g.n_layers = n_layers;
  g.n_kv_heads = n_kv_heads;
  g.head_dim = head_dim;
  g.capacity = capacity;
  g.elem = elem;
  g.kv_dim = n_kv_heads * head_dim;
  const size_t ws = std::max<size_t>(rv::decode_ws_bound(&g), (size_t)1 << 20);
  const size_t staged = n_layers * rv::prefill_stage_bound(&g);
  const size_t tab = capacity * head_dim * sizeof(float);
  *bytes = planes + ws + rv::ticket_words(&g) * sizeof(unsigned) + staged + tab;
  return ok(err);
}

int32_t rv_kv_xcd_dealing(rv_kv* kv, int32_t* ok_out, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  if (!ok_out) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "ok");
  *ok_out = kv->xcd_ok ? 1 : 0;
  return ok(err);
}

int32_t rv_position_advance(rv_kv* kv, uint32_t* d_position, uint32_t n, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  if (!d_position) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "d_position");
  DeviceGuard dg(kv->device);
  const rv::HipStatus hs = rv::launch_position_advance(d_position, n, kv->stream);
  if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  return ok(err);
}

// model/prefill.rs:2055-2111 steps (d)-(f).
int32_t rv_prefill_chunk(rv_kv* kv, size_t layer, const float* q_rows, const float* k_rows, const float* v_rows,
                         size_t rows, size_t q_dim, const float* q_norm_w, size_t q_norm_len, const float* k_norm_w,
                         size_t k_norm_len, float eps, float theta, size_t start, float scale, float* out,
                         uint32_t flags, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  int32_t rc = check_rope_dim(kv, err);
  if (rc) return rc;
  const size_t hd = kv->head_dim;
  if (q_dim == 0 || q_dim % hd) return fail(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_dim, hd);
  if ((q_dim / hd) % kv->n_kv_heads) return fail(err, RV_ATTN_GQA_GROUP_MISMATCH, q_dim / hd, kv->n_kv_heads);
  if (rows > 0 && (rc = check_norm_weights(hd, q_norm_len, k_norm_len, err))) return rc;
  if ((rc = check_layer(kv, layer, err))) return rc;
  const size_t len = kv->lens[layer];
  if (start != len) return fail(err, RV_KV_POSITION_OUT_OF_RANGE, layer, start, len, 0, "start != len(layer)");
  if (rows > kv->capacity - len) return fail(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity);
  if (start + rows > 0x100000000ull) return fail(err, RV_ERR_UNSUPPORTED, start + rows, 0, 0, 0, "position past u32");
  if (rows == 0) return ok(err);
  if (!q_rows || !k_rows || !v_rows || !q_norm_w || !k_norm_w || !out)
    return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "tensor");
  DeviceGuard dg(kv->device);
  const size_t nq = rows * q_dim, nk = rows * kv->kv_dim;
  const float *dq = q_rows, *dk = k_rows, *dv = v_rows, *dwq = q_norm_w, *dwk = k_norm_w;
  float* dout = out;
  if (flags & RV_HOST_PTRS) {
    Stager st(kv);
    const size_t need = 2 * Stager::align(nq * 4) + 2 * Stager::align(nk * 4) + 2 * Stager::align(hd * 4);
    if (!st.reserve(need)) return hip_fail(err, st.e, "hipMalloc stage");
    dq = st.in(q_rows, nq);
    dk = st.in(k_rows, nk);
    dv = st.in(v_rows, nk);
    dwq = st.in(q_norm_w, hd);
    dwk = st.in(k_norm_w, hd);
    dout = st.carve(nq);
    if (st.e != hipSuccess) return hip_fail(err, st.e, "hipMemcpyAsync H2D");
  }
  rv::InvFreq inv;
  rv::fill_inv_freq(inv, hd, theta);
  Plan p{q_dim / hd, q_dim / hd / kv->n_kv_heads, 0};
  rv::HipStatus hs;
  if (rv::prefill_supported(kv, p.group, start + rows)) {
    // k/v prologue + append, also into the layer's staged tiles. Where the
    // chunk's rows are staged as they are appended (F16 / BF16, uncaptured),
    // the same launch writes the q heads in the attention kernel's prepared
    // layout; otherwise it writes the rows' (cos, sin) table and the q
    // prologue runs inside the attention kernel's query loads.
    rv::StageDst sd;
    hs = rv::prepare_prefill_stage(kv, layer, len, rows, flags, kv->stream, &sd);
    // (The preparation reads q and its norm weight with 16-byte loads.)
    const bool prep = sd.base != nullptr && ((uintptr_t)dq % 16) == 0 && ((uintptr_t)dwq % 16) == 0 &&
                      q_dim % 4 == 0;
    const int vectors = prep ? rv::prefill_vectors(kv, rows, start, p.group) : 0;
    if (hs.e == hipSuccess)
      hs = rv::ensure_qbuf(kv, prep ? rv::qprep_bytes(rows, kv->n_kv_heads, p.group, vectors)
                                    : rows * hd * sizeof(float));
    rv::QPrep qp = prep ? rv::qprep_plan((char*)kv->qbuf, rows, p.group, scale, vectors) : rv::QPrep{};
    if (prep && hs.e == hipSuccess) {
      hs = rv::ensure_rope_tab(kv, theta, start + rows);
      qp.rope = kv->rope_tab;
    }
    if (hs.e == hipSuccess)
      hs = rv::launch_row_prologue(kv, layer, len, prep ? dq : nullptr, nullptr, prep ? p.n_q_heads : 0, dk, dv, rows,
                                   prep ? dwq : nullptr, dwk, eps, inv, start, prep ? nullptr : kv->qbuf, &sd,
                                   kv->stream, prep ? &qp : nullptr);
    if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
    kv->lens[layer] = len + rows;
    rv::QNorm qn{dwq, eps, kv->qbuf};
    if (prep) qn.prepped = (const char*)kv->qbuf;
    hs = rv::launch_prefill(kv, dq, rows, p.n_q_heads, layer, start, scale, dout, flags, &qn, kv->stream);
    if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
  } else {
    hs = rv::ensure_qbuf(kv, nq * sizeof(float));
    if (hs.e == hipSuccess)
      hs = rv::launch_row_prologue(kv, layer, len, dq, kv->qbuf, q_dim / hd, dk, dv, rows, dwq, dwk, eps, inv, start,
                                   nullptr, nullptr, kv->stream);
    if (hs.e != hipSuccess) return hip_fail(err, hs.e, hs.what);
    kv->lens[layer] = len + rows;
    rc = run_rows(kv, kv->qbuf, rows, q_dim, layer, start, p, scale, dout, flags, err);
    if (rc) return rc;
  }
  return finish(kv, flags, dout, out, nq, err);
}

int32_t rv_kv_set_tuning(rv_kv* kv, int32_t knob, int64_t value, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  switch (knob) {
    case RV_TUNE_DECODE_SPLIT_LEN: kv->tune_decode_split_len = value; break;
    case RV_TUNE_PREFILL_KV_SPLIT: kv->tune_prefill_kv_split = value; break;
    case RV_TUNE_DECODE_WAVES: kv->tune_decode_waves = value; break;
    case RV_TUNE_PREFILL_ROWS: kv->tune_prefill_rows = value; break;
    case RV_TUNE_DECODE_HG: kv->tune_decode_hg = value; break;
    case RV_TUNE_DECODE_IMPL: kv->tune_decode_impl = value; break;
    case RV_TUNE_KERNEL_TIMING: kv->timing = value != 0; break;
    case RV_TUNE_DECODE_DEPTH: kv->tune_decode_depth = value; break;
    case RV_TUNE_DECODE_MERGE: kv->tune_decode_merge = value; break;
    default: return fail(err, RV_ERR_UNSUPPORTED, (uint64_t)knob, 0, 0, 0, "tuning knob");
  }
  return ok(err);
}

int32_t rv_kv_kernel_time(rv_kv* kv, double* total_ms, uint64_t* launches, rv_error* err) {
  if (!kv) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, "kv");
  if (!total_ms || !launches) return fail(err, RV_ERR_NULL_ARG, 0, 0, 0, 0, !total_ms ? "total_ms" : "launches");
  DeviceGuard dg(kv->device);
  const hipError_t e = kv->stream ? hipStreamSynchronize(kv->stream) : hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(err, e, "synchronize before reading kernel times");
  rv::timing_fold(kv);
  *total_ms = kv->timed_ms;
  *launches = kv->timed_n;
  kv->timed_ms = 0;
  kv->timed_n = 0;
  return ok(err);
}

}  // extern "C"
