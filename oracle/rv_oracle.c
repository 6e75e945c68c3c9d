/*
 * rv_oracle.c — CPU restatement of ramvamp's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline. Citations are `path:line` into ramvamp's crates/core/src.
 * Build with -O2 -ffp-contract=off -fno-fast-math (oracle/Makefile): every
 * f32 multiply and add below must round separately, as Rust's do.
 *
 * Parity pinning of each part lives in tests/test_oracle.py (known-answer
 * vectors from the reference's own tests, closed forms, f64 textbook
 * attention and the reference's internal bit-identity gates).
 */
#define _GNU_SOURCE
#include "rv_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static int32_t set_err(rv_error* err, int32_t code, uint64_t a, uint64_t b, uint64_t c,
                       uint64_t d, const char* what) {
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

/* ---- f16 (kernels/quants/f16.rs) -------------------------------------- */

static float f32_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* f16.rs:17-32: exact widening. */
float rvo_f16_to_f32(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits >> 15) << 31;
  uint32_t exp = (bits >> 10) & 0x1F;
  uint32_t frac = bits & 0x03FF;
  if (exp == 0) {
    /* frac * 2^-24 is exact in f32 (f16.rs:9-10, 0x3380_0000 = 2^-24). */
    float magnitude = (float)frac * f32_from_bits(0x33800000u);
    return f32_from_bits(f32_bits(magnitude) | sign);
  }
  if (exp == 0x1F) return f32_from_bits(sign | 0x7F800000u | (frac << 13));
  return f32_from_bits(sign | ((exp + 112u) << 23) | (frac << 13));
}

/* f16.rs:39-91: round to nearest, ties to even; subnormals, inf, NaN. */
uint16_t rvo_f32_to_f16(float x) {
  uint32_t bits = f32_bits(x);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  int32_t exp = (int32_t)((bits >> 23) & 0xFF);
  uint32_t frac = bits & 0x007FFFFFu;
  if (exp == 0xFF) {
    if (frac == 0) return sign | 0x7C00;
    return sign | 0x7C00 | 0x0200 | ((uint16_t)(frac >> 13) & 0x03FF);
  }
  int32_t e16 = exp - 112;
  if (e16 >= 0x1F) return sign | 0x7C00;
  if (e16 <= 0) {
    if (e16 < -10) return sign;
    uint32_t mant = exp == 0 ? frac : (frac | 0x00800000u);
    uint32_t shift = (uint32_t)(14 - e16);
    uint32_t ulp = 1u << shift;
    uint32_t half = ulp >> 1;
    uint32_t v = mant >> shift;
    uint32_t rem = mant & (ulp - 1);
    if (rem > half || (rem == half && (v & 1))) v += 1;
    return sign | (uint16_t)v;
  }
  uint32_t v = ((uint32_t)e16 << 10) | (frac >> 13);
  uint32_t rem = frac & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (v & 1))) v += 1;
  return sign | (uint16_t)v;
}

void rvo_f16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = rvo_f16_to_f32(src[i]);
}
void rvo_f32_to_f16_n(const float* src, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = rvo_f32_to_f16(src[i]);
}

/* ---- KV cache (kv/mod.rs) --------------------------------------------- */

static size_t elem_size(int elem) { return elem == RV_ELEM_F32 ? 4 : 2; }

/* kv/mod.rs:190-231 `geometry`: nonzero dims, checked products. */
static int32_t geometry(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity,
                        size_t* kv_dim, size_t* plane, size_t* total, rv_error* err) {
#define INVALID(reason) \
  set_err(err, RV_KV_INVALID_DIMS, n_layers, n_kv_heads, head_dim, capacity, reason)
  if (n_layers == 0 || n_kv_heads == 0 || head_dim == 0 || capacity == 0)
    return INVALID("all dims must be nonzero");
  size_t a;
  if (__builtin_mul_overflow(n_kv_heads, head_dim, &a)) return INVALID("row width overflows usize");
  *kv_dim = a;
  if (__builtin_mul_overflow(capacity, *kv_dim, &a)) return INVALID("plane size overflows usize");
  *plane = a;
  if (__builtin_mul_overflow(n_layers, *plane, &a)) return INVALID("total size overflows usize");
  *total = a;
  return RV_OK;
#undef INVALID
}

/* kv/mod.rs:237-259. */
int32_t rvo_kv_projected_bytes(size_t n_layers, size_t n_kv_heads, size_t head_dim,
                               size_t capacity, int elem, uint64_t* bytes, rv_error* err) {
  size_t kv_dim, plane, total, b2, b;
  int32_t rc = geometry(n_layers, n_kv_heads, head_dim, capacity, &kv_dim, &plane, &total, err);
  if (rc) return rc;
  if (__builtin_mul_overflow(total, (size_t)2, &b2) ||
      __builtin_mul_overflow(b2, elem_size(elem), &b))
    return set_err(err, RV_KV_INVALID_DIMS, n_layers, n_kv_heads, head_dim, capacity,
                   "total size in bytes overflows usize");
  *bytes = (uint64_t)b;
  return RV_OK;
}

/* kv/mod.rs:163-181. */
int32_t rvo_kv_new(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity,
                   int elem, rvo_kv** out, rv_error* err) {
  if (elem != RV_ELEM_F16 && elem != RV_ELEM_F32)
    return set_err(err, RV_ERR_BAD_ELEM, (uint64_t)elem, 0, 0, 0, "elem");
  size_t kv_dim, plane, total;
  int32_t rc = geometry(n_layers, n_kv_heads, head_dim, capacity, &kv_dim, &plane, &total, err);
  if (rc) return rc;
  rvo_kv* kv = calloc(1, sizeof *kv);
  kv->n_layers = n_layers;
  kv->n_kv_heads = n_kv_heads;
  kv->head_dim = head_dim;
  kv->capacity = capacity;
  kv->kv_dim = kv_dim;
  kv->plane = plane;
  kv->elem = elem;
  kv->k = calloc(total, elem_size(elem));
  kv->v = calloc(total, elem_size(elem));
  kv->lens = calloc(n_layers, sizeof(size_t));
  if (!kv->k || !kv->v || !kv->lens) {
    rvo_kv_free(kv);
    return set_err(err, RV_KV_INVALID_DIMS, n_layers, n_kv_heads, head_dim, capacity,
                   "host allocation failed");
  }
  *out = kv;
  return RV_OK;
}

void rvo_kv_free(rvo_kv* kv) {
  if (!kv) return;
  free(kv->k);
  free(kv->v);
  free(kv->lens);
  free(kv);
}

/* kv/mod.rs:462-470 `check_layer`. */
static int32_t check_layer(const rvo_kv* kv, size_t layer, rv_error* err) {
  if (layer >= kv->n_layers)
    return set_err(err, RV_KV_LAYER_OUT_OF_RANGE, layer, kv->n_layers, 0, 0, NULL);
  return RV_OK;
}

int32_t rvo_kv_len(const rvo_kv* kv, size_t layer, size_t* len, rv_error* err) {
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  *len = kv->lens[layer];
  return RV_OK;
}

int rvo_kv_is_empty(const rvo_kv* kv) {
  for (size_t l = 0; l < kv->n_layers; ++l)
    if (kv->lens[l]) return 0;
  return 1;
}

/* kv/mod.rs:312-325. */
int32_t rvo_kv_seq_len(const rvo_kv* kv, size_t* len, rv_error* err) {
  size_t lo = SIZE_MAX, hi = 0;
  for (size_t l = 0; l < kv->n_layers; ++l) {
    if (kv->lens[l] < lo) lo = kv->lens[l];
    if (kv->lens[l] > hi) hi = kv->lens[l];
  }
  if (lo != hi) return set_err(err, RV_KV_RAGGED_LAYERS, lo, hi, 0, 0, NULL);
  *len = lo;
  return RV_OK;
}

/* kv/mod.rs:336-368: layer, k length, v length, capacity — in that order. */
int32_t rvo_kv_append(rvo_kv* kv, size_t layer, const float* k, size_t k_len, const float* v,
                      size_t v_len, rv_error* err) {
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  if (k_len != kv->kv_dim) return set_err(err, RV_KV_ROW_LEN_MISMATCH, k_len, kv->kv_dim, 0, 0, "k");
  if (v_len != kv->kv_dim) return set_err(err, RV_KV_ROW_LEN_MISMATCH, v_len, kv->kv_dim, 0, 0, "v");
  size_t len = kv->lens[layer];
  if (len == kv->capacity)
    return set_err(err, RV_KV_CAPACITY_EXCEEDED, layer, kv->capacity, 0, 0, NULL);
  size_t base = layer * kv->plane + len * kv->kv_dim;
  if (kv->elem == RV_ELEM_F16) {
    uint16_t* kd = (uint16_t*)kv->k + base;
    uint16_t* vd = (uint16_t*)kv->v + base;
    for (size_t i = 0; i < kv->kv_dim; ++i) kd[i] = rvo_f32_to_f16(k[i]);
    for (size_t i = 0; i < kv->kv_dim; ++i) vd[i] = rvo_f32_to_f16(v[i]);
  } else {
    memcpy((float*)kv->k + base, k, kv->kv_dim * 4);
    memcpy((float*)kv->v + base, v, kv->kv_dim * 4);
  }
  kv->lens[layer] = len + 1;
  return RV_OK;
}

/* kv/mod.rs:383-385. */
void rvo_kv_clear(rvo_kv* kv) { memset(kv->lens, 0, kv->n_layers * sizeof(size_t)); }

/* kv/mod.rs:410-420: ragged refused first, then an upward target. */
int32_t rvo_kv_truncate(rvo_kv* kv, size_t new_len, rv_error* err) {
  size_t len;
  int32_t rc = rvo_kv_seq_len(kv, &len, err);
  if (rc) return rc;
  if (new_len > len) return set_err(err, RV_KV_TRUNCATE_BEYOND_LENGTH, new_len, len, 0, 0, NULL);
  for (size_t l = 0; l < kv->n_layers; ++l) kv->lens[l] = new_len;
  return RV_OK;
}

/* kv/mod.rs:472-480 `row`. */
int32_t rvo_kv_read_row(const rvo_kv* kv, int plane_v, size_t layer, size_t pos, void* dst,
                        rv_error* err) {
  int32_t rc = check_layer(kv, layer, err);
  if (rc) return rc;
  size_t len = kv->lens[layer];
  if (pos >= len) return set_err(err, RV_KV_POSITION_OUT_OF_RANGE, layer, pos, len, 0, NULL);
  size_t es = elem_size(kv->elem);
  const char* plane = (const char*)(plane_v ? kv->v : kv->k);
  memcpy(dst, plane + (layer * kv->plane + pos * kv->kv_dim) * es, kv->kv_dim * es);
  return RV_OK;
}

/* ---- primitives -------------------------------------------------------- */

/* primitives/softmax.rs:18-40: max in f32, exp and sum in f64, multiply by
 * the f32-rounded reciprocal. */
int32_t rvo_softmax(float* x, size_t n) {
  if (n == 0) return RV_PRIM_LENGTH_MISMATCH;
  float max = -INFINITY;
  for (size_t i = 0; i < n; ++i)
    if (x[i] > max) max = x[i];
  double m = (double)max;
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    double e = exp((double)x[i] - m);
    x[i] = (float)e;
    sum += e;
  }
  float inv = (float)(1.0 / sum);
  for (size_t i = 0; i < n; ++i) x[i] *= inv;
  return RV_OK;
}

/* primitives/norm.rs:18-26 `inv_rms`: f64 mean of squares. */
static float inv_rms(const float* x, size_t n, float eps) {
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    double v = (double)x[i];
    sum += v * v;
  }
  double mean = sum / (double)n;
  return (float)(1.0 / sqrt(mean + (double)eps));
}

/* primitives/norm.rs:72-90: `v * inv * w`, left to right in f32. */
int32_t rvo_rmsnorm_in_place(float* x, const float* w, size_t n, float eps) {
  if (n == 0) return RV_PRIM_LENGTH_MISMATCH;
  float inv = inv_rms(x, n, eps);
  for (size_t i = 0; i < n; ++i) x[i] = x[i] * inv * w[i];
  return RV_OK;
}

/* primitives/rope.rs:31-45 `rotate_head`: f64 angle and sin/cos, rotation
 * applied in f32 with separate multiply and subtract/add. */
static void rotate_head(float* head, size_t half, uint32_t position, float theta_base) {
  double pos = (double)position;
  double base = (double)theta_base;
  double dim = (double)(2 * half);
  for (size_t i = 0; i < half; ++i) {
    double inv_freq = pow(base, -2.0 * (double)i / dim);
    double angle = pos * inv_freq;
    float s = (float)sin(angle), c = (float)cos(angle);
    float x0 = head[i], x1 = head[i + half];
    head[i] = x0 * c - x1 * s;
    head[i + half] = x0 * s + x1 * c;
  }
}

/* primitives/rope.rs:82-105. */
int32_t rvo_rope_neox_heads(float* x, size_t x_len, size_t n_heads, size_t head_dim,
                            uint32_t position, float theta) {
  if (head_dim == 0 || head_dim % 2) return RV_PRIM_INVALID_HEAD_DIM;
  size_t expected;
  if (__builtin_mul_overflow(n_heads, head_dim, &expected) || expected != x_len)
    return RV_PRIM_LENGTH_MISMATCH;
  for (size_t h = 0; h < n_heads; ++h) rotate_head(x + h * head_dim, head_dim / 2, position, theta);
  return RV_OK;
}

int32_t rvo_norm_rope_heads(float* x, size_t n_heads, size_t head_dim, const float* w,
                            float eps, float theta, uint32_t position) {
  for (size_t h = 0; h < n_heads; ++h) {
    int32_t rc = rvo_rmsnorm_in_place(x + h * head_dim, w, head_dim, eps);
    if (rc) return rc;
  }
  return rvo_rope_neox_heads(x, n_heads * head_dim, n_heads, head_dim, position, theta);
}

/* ---- attention (kernels/attention.rs) ---------------------------------- */

/* attention.rs:337-359, saturating. */
static size_t sat_mul(size_t a, size_t b) {
  size_t r;
  return __builtin_mul_overflow(a, b, &r) ? SIZE_MAX : r;
}
static size_t sat_add(size_t a, size_t b) {
  size_t r;
  return __builtin_add_overflow(a, b, &r) ? SIZE_MAX : r;
}
static size_t scratch_len_of(size_t group, size_t head_dim, size_t max_positions) {
  return sat_add(sat_mul(group, max_positions), sat_mul(head_dim, 2));
}
size_t rvo_scratch_len(size_t n_q_heads, size_t n_kv_heads, size_t head_dim,
                       size_t max_positions) {
  size_t group = n_kv_heads ? n_q_heads / n_kv_heads : 0;
  return scratch_len_of(group, head_dim, max_positions);
}

typedef struct plan_t {
  size_t head_dim, kv_dim, group, positions, kv_lo, kv_hi;
} plan_t;

/* attention.rs:926-989 `plan`: q, GQA, layer, positions, kv range, out. */
static int32_t plan(const float* q, size_t q_len, const rvo_kv* kv, size_t layer, int has_limit,
                    size_t limit, size_t kv_lo, size_t kv_hi, size_t out_len, plan_t* p,
                    rv_error* err) {
  (void)q;
  size_t head_dim = kv->head_dim, n_kv = kv->n_kv_heads;
  if (q_len == 0 || q_len % head_dim)
    return set_err(err, RV_ATTN_Q_LEN_INDIVISIBLE, q_len, head_dim, 0, 0, NULL);
  size_t n_q = q_len / head_dim;
  if (n_q % n_kv) return set_err(err, RV_ATTN_GQA_GROUP_MISMATCH, n_q, n_kv, 0, 0, NULL);
  size_t len;
  int32_t rc = rvo_kv_len(kv, layer, &len, err);
  if (rc) return rc;
  size_t positions = has_limit ? limit : len;
  if (positions == 0) return set_err(err, RV_ATTN_EMPTY_LAYER, layer, 0, 0, 0, NULL);
  if (positions > len)
    return set_err(err, RV_KV_POSITION_OUT_OF_RANGE, layer, positions - 1, len, 0, NULL);
  if (kv_lo > kv_hi || kv_hi > n_kv)
    return set_err(err, RV_ATTN_KV_HEAD_RANGE, kv_lo, kv_hi, n_kv, 0, NULL);
  size_t group = n_q / n_kv;
  size_t expected = (kv_hi - kv_lo) * group * head_dim;
  if (out_len != expected) return set_err(err, RV_ATTN_OUT_LEN_MISMATCH, out_len, expected, 0, 0, NULL);
  p->head_dim = head_dim;
  p->kv_dim = kv->kv_dim;
  p->group = group;
  p->positions = positions;
  p->kv_lo = kv_lo;
  p->kv_hi = kv_hi;
  return RV_OK;
}

/* One K/V head slice widened to f32: f16 bits through the exact integer
 * conversion, or f32 copied (the fp32-element planes). */
static void widen_scalar(const rvo_kv* kv, const void* plane, size_t idx, float* dst, size_t n) {
  if (kv->elem == RV_ELEM_F16) {
    const uint16_t* src = (const uint16_t*)plane + idx;
    for (size_t i = 0; i < n; ++i) dst[i] = rvo_f16_to_f32(src[i]);
  } else {
    memcpy(dst, (const float*)plane + idx, n * 4);
  }
}

/* attention.rs:1212-1239 `qk_scores_scalar`. */
static void qk_scores_scalar(const rvo_kv* kv, const float* q_group, const void* k_layer,
                             size_t kv_dim, size_t col, size_t head_dim, size_t group,
                             size_t positions, float scale, float* kbuf, float* scores) {
  for (size_t t = 0; t < positions; ++t) {
    widen_scalar(kv, k_layer, t * kv_dim + col, kbuf, head_dim);
    for (size_t g = 0; g < group; ++g) {
      const float* q_h = q_group + g * head_dim;
      float acc = 0.0f;
      for (size_t i = 0; i < head_dim; ++i) acc += q_h[i] * kbuf[i];
      scores[g * positions + t] = scale * acc;
    }
  }
}

/* attention.rs:1278-1303 `v_reduce_scalar`. */
static void v_reduce_scalar(const rvo_kv* kv, const void* v_layer, size_t kv_dim, size_t col,
                            size_t head_dim, size_t group, size_t positions,
                            const float* scores, float* vbuf, float* out_group) {
  for (size_t t = 0; t < positions; ++t) {
    widen_scalar(kv, v_layer, t * kv_dim + col, vbuf, head_dim);
    for (size_t g = 0; g < group; ++g) {
      float w = scores[g * positions + t];
      float* o = out_group + g * head_dim;
      for (size_t i = 0; i < head_dim; ++i) o[i] += w * vbuf[i];
    }
  }
}

/* ---- AVX2 + F16C body (kernels/attention/x86.rs) ----------------------- */

#define LANES 8           /* x86.rs:97 */
#define T_BLOCK 8         /* x86.rs:138 */
#define T_TAIL_BLOCK 4    /* x86.rs:165 */
#define MAX_SIMD_HEAD_DIM 256 /* attention.rs:158 */

int rvo_avx2_path_covers(size_t head_dim) {
  return head_dim <= MAX_SIMD_HEAD_DIM && __builtin_cpu_supports("avx2") &&
         __builtin_cpu_supports("f16c");
}

/* x86.rs:193-211 `widen`: eight at a time through vcvtph2ps (exact), the
 * tail through the integer conversion. The f32-element plane copies. */
__attribute__((target("avx2,f16c"))) static void widen_avx(const rvo_kv* kv, const void* plane,
                                                           size_t idx, float* dst, size_t n) {
  if (kv->elem != RV_ELEM_F16) {
    memcpy(dst, (const float*)plane + idx, n * 4);
    return;
  }
  const uint16_t* src = (const uint16_t*)plane + idx;
  size_t i = 0;
  for (; i + LANES <= n; i += LANES) {
    __m128i half = _mm_loadu_si128((const __m128i*)(src + i));
    _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(half));
  }
  for (; i < n; ++i) dst[i] = rvo_f16_to_f32(src[i]);
}

/* x86.rs:257-286 `dot_block`: lanes over the group, i ascending, separate
 * multiply and add, scale applied after the dot. */
__attribute__((target("avx2,f16c"))) static void dot_block(const float* qt, const float* kb,
                                                           size_t head_dim, float scale, int n,
                                                           float out[][LANES]) {
  __m256 acc[T_BLOCK];
  for (int j = 0; j < n; ++j) acc[j] = _mm256_setzero_ps();
  for (size_t i = 0; i < head_dim; ++i) {
    __m256 qv = _mm256_loadu_ps(qt + i * LANES);
    for (int j = 0; j < n; ++j) {
      __m256 kv = _mm256_broadcast_ss(kb + (size_t)j * head_dim + i);
      acc[j] = _mm256_add_ps(acc[j], _mm256_mul_ps(qv, kv));
    }
  }
  __m256 s = _mm256_set1_ps(scale);
  for (int j = 0; j < n; ++j) _mm256_storeu_ps(out[j], _mm256_mul_ps(s, acc[j]));
}

/* x86.rs:366-434 `qk_scores`: group chunks of LANES, position blocks of
 * T_BLOCK, one T_TAIL_BLOCK rung, then single positions. */
__attribute__((target("avx2,f16c"))) static void qk_scores_avx(
    const rvo_kv* kv, const float* q_group, const void* k_layer, size_t kv_dim, size_t col,
    size_t head_dim, size_t group, size_t positions, float scale, float* scores) {
  float qt[LANES * MAX_SIMD_HEAD_DIM];
  float kb[T_BLOCK * MAX_SIMD_HEAD_DIM];
  float block[T_BLOCK][LANES];
  for (size_t base = 0; base < group; base += LANES) {
    size_t lanes = group - base < LANES ? group - base : LANES;
    for (size_t g = 0; g < LANES; ++g)
      for (size_t i = 0; i < head_dim; ++i)
        qt[i * LANES + g] = g < lanes ? q_group[(base + g) * head_dim + i] : 0.0f;
    size_t t = 0;
    int rungs[3] = {T_BLOCK, T_TAIL_BLOCK, 1};
    for (int r = 0; r < 3; ++r) {
      int n = rungs[r];
      /* main block loops; the tail rung fires at most once; singles loop */
      while (t + (size_t)n <= positions) {
        for (int j = 0; j < n; ++j) widen_avx(kv, k_layer, (t + j) * kv_dim + col, kb + j * head_dim, head_dim);
        dot_block(qt, kb, head_dim, scale, n, block);
        for (int j = 0; j < n; ++j)
          for (size_t g = 0; g < lanes; ++g) scores[(base + g) * positions + t + j] = block[j][g];
        t += n;
        if (n == T_TAIL_BLOCK) break;
      }
    }
  }
}

/* x86.rs:449-490 `v_reduce`: lanes over i, t sequential. */
__attribute__((target("avx2,f16c"))) static void v_reduce_avx(
    const rvo_kv* kv, const void* v_layer, size_t kv_dim, size_t col, size_t head_dim,
    size_t group, size_t positions, const float* scores, float* vbuf, float* out_group) {
  for (size_t t = 0; t < positions; ++t) {
    widen_avx(kv, v_layer, t * kv_dim + col, vbuf, head_dim);
    for (size_t g = 0; g < group; ++g) {
      float w = scores[g * positions + t];
      float* o = out_group + g * head_dim;
      __m256 wv = _mm256_set1_ps(w);
      size_t i = 0;
      for (; i + LANES <= head_dim; i += LANES) {
        __m256 ov = _mm256_loadu_ps(o + i);
        __m256 vv = _mm256_loadu_ps(vbuf + i);
        _mm256_storeu_ps(o + i, _mm256_add_ps(ov, _mm256_mul_ps(wv, vv)));
      }
      for (; i < head_dim; ++i) o[i] += w * vbuf[i];
    }
  }
}

/* attention.rs:1075-1160 `attention_body`: kv head outer, group inner. */
static int32_t attention_body(const float* q, const rvo_kv* kv, size_t layer, const plan_t* p,
                              float scale, float* scratch, float* out, int force_scalar) {
  size_t es = elem_size(kv->elem);
  const void* k_layer = (const char*)kv->k + layer * kv->plane * es;
  const void* v_layer = (const char*)kv->v + layer * kv->plane * es;
  size_t positions = p->positions, head_dim = p->head_dim, group = p->group;
  float* scores = scratch;
  float* kbuf = scratch + group * positions;
  float* vbuf = kbuf + head_dim;
  size_t group_dim = group * head_dim;
  int simd = !force_scalar && rvo_avx2_path_covers(head_dim);
  for (size_t kv_head = p->kv_lo, c = 0; kv_head < p->kv_hi; ++kv_head, ++c) {
    const float* q_group = q + kv_head * group_dim;
    float* out_group = out + c * group_dim;
    size_t col = kv_head * head_dim;
    if (simd)
      qk_scores_avx(kv, q_group, k_layer, p->kv_dim, col, head_dim, group, positions, scale, scores);
    else
      qk_scores_scalar(kv, q_group, k_layer, p->kv_dim, col, head_dim, group, positions, scale,
                       kbuf, scores);
    for (size_t g = 0; g < group; ++g) rvo_softmax(scores + g * positions, positions);
    memset(out_group, 0, group_dim * 4);
    if (simd)
      v_reduce_avx(kv, v_layer, p->kv_dim, col, head_dim, group, positions, scores, vbuf, out_group);
    else
      v_reduce_scalar(kv, v_layer, p->kv_dim, col, head_dim, group, positions, scores, vbuf,
                      out_group);
  }
  return RV_OK;
}

/* attention_owned (attention.rs:993-1020) when scratch is NULL, else
 * attention_borrowed (attention.rs:1022-1045). */
int32_t rvo_attention(const float* q, size_t q_len, const rvo_kv* kv, size_t layer,
                      int has_limit, size_t limit, float scale, size_t kv_lo, size_t kv_hi,
                      float* scratch, size_t scratch_len, float* out, size_t out_len,
                      int force_scalar, rv_error* err) {
  plan_t p;
  int32_t rc = plan(q, q_len, kv, layer, has_limit, limit, kv_lo, kv_hi, out_len, &p, err);
  if (rc) return rc;
  if (scratch) {
    size_t need = scratch_len_of(p.group, p.head_dim, p.positions);
    if (scratch_len < need) return set_err(err, RV_ATTN_SCRATCH_TOO_SHORT, scratch_len, need, 0, 0, NULL);
    return attention_body(q, kv, layer, &p, scale, scratch, out, force_scalar);
  }
  size_t cap = kv->capacity > p.positions ? kv->capacity : p.positions;
  size_t need = scratch_len_of(p.group, p.head_dim, cap);
  float* buf = calloc(need, 4);
  rc = attention_body(q, kv, layer, &p, scale, buf, out, force_scalar);
  free(buf);
  return rc;
}

/* ---- fan-out policies --------------------------------------------------- */

/* forward.rs:2057-2060 `first(u)`: slot u's first kv head. */
static size_t slot_first(size_t u, size_t units, size_t base, size_t rem) {
  if (u > units) u = units;
  return u * base + (u < rem ? u : rem);
}

/* model/forward.rs:2052-2063. */
void rvo_kv_head_range(size_t n_kv_heads, size_t units, size_t slot_lo, size_t slot_hi,
                       size_t* lo, size_t* hi) {
  if (units == 0) {
    *lo = *hi = 0;
    return;
  }
  size_t base = n_kv_heads / units, rem = n_kv_heads % units;
  size_t l = slot_first(slot_lo, units, base, rem), h = slot_first(slot_hi, units, base, rem);
  *lo = l;
  *hi = h > l ? h : l;
}

/* model/prefill.rs:1211-1214. */
static unsigned __int128 attention_cost(size_t rows, size_t start) {
  unsigned __int128 r = rows;
  return r * start + r * (r + 1) / 2;
}

/* model/prefill.rs:1257-1281: smallest row whose cost reaches the target. */
static size_t attention_boundary(size_t rows, size_t start, unsigned __int128 total,
                                 size_t shards, size_t index) {
  if (index == 0) return 0;
  if (index >= shards) return rows;
  unsigned __int128 target = total * index / shards;
  size_t lo = 0, hi = rows;
  while (lo < hi) {
    size_t mid = lo + (hi - lo) / 2;
    if (attention_cost(mid, start) < target)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

/* model/prefill.rs:1238-1250. */
void rvo_attention_shard_range(size_t rows, size_t start, size_t shards, size_t index,
                               size_t* lo, size_t* hi) {
  if (shards == 0 || index >= shards) {
    *lo = *hi = 0;
    return;
  }
  if (shards == 1) {
    *lo = 0;
    *hi = rows;
    return;
  }
  unsigned __int128 total = attention_cost(rows, start);
  *lo = attention_boundary(rows, start, total, shards, index);
  *hi = attention_boundary(rows, start, total, shards, index + 1);
}

/* ---- threaded callers (the CPU baseline) -------------------------------- */

typedef struct decode_job {
  const rvo_kv* kv;
  size_t layer, q_len, lo, hi, group_dim;
  float scale;
  const float* q;
  float* out;
  int force_scalar;
  int32_t rc;
  rv_error err;
} decode_job;

static void* decode_worker(void* arg) {
  decode_job* j = arg;
  size_t n_q = j->q_len / j->kv->head_dim;
  size_t need = rvo_scratch_len(n_q, j->kv->n_kv_heads, j->kv->head_dim, j->kv->capacity);
  float* scratch = malloc(need * 4);
  j->rc = rvo_attention(j->q, j->q_len, j->kv, j->layer, 0, 0, j->scale, j->lo, j->hi, scratch,
                        need, j->out + j->lo * j->group_dim, (j->hi - j->lo) * j->group_dim,
                        j->force_scalar, &j->err);
  free(scratch);
  return NULL;
}

/* model/forward.rs:1914-2031: serial below ATTENTION_FANOUT_MIN_POSITIONS
 * (forward.rs:1784) or on any shape the split cannot tile; else one kv-head
 * range per shard (kv_head_range over `units` slots). */
int32_t rvo_pool_decode_attention(const rvo_kv* kv, size_t layer, float scale, const float* q,
                                  size_t q_len, float* out, size_t out_len, size_t threads,
                                  int force_scalar, rv_error* err) {
  size_t n_kv = kv->n_kv_heads, units = threads;
  size_t positions = layer < kv->n_layers ? kv->lens[layer] : 0;
  size_t group_dim = n_kv ? q_len / n_kv : 0;
  if (units < 2 || n_kv < 2 || positions < 8 || out_len != q_len || group_dim == 0 ||
      group_dim * n_kv != q_len) {
    size_t n_q = kv->head_dim ? q_len / kv->head_dim : 0;
    size_t need = rvo_scratch_len(n_q, n_kv, kv->head_dim, kv->capacity);
    float* scratch = malloc((need ? need : 1) * 4);
    int32_t rc = rvo_attention(q, q_len, kv, layer, 0, 0, scale, 0, n_kv, scratch, need, out,
                               out_len, force_scalar, err);
    free(scratch);
    return rc;
  }
  decode_job* jobs = calloc(units, sizeof *jobs);
  pthread_t* tid = calloc(units, sizeof *tid);
  int* started = calloc(units, sizeof *started);
  for (size_t u = 0; u < units; ++u) {
    decode_job* j = &jobs[u];
    rvo_kv_head_range(n_kv, units, u, u + 1, &j->lo, &j->hi);
    if (j->lo == j->hi) continue;
    j->kv = kv;
    j->layer = layer;
    j->q_len = q_len;
    j->group_dim = group_dim;
    j->scale = scale;
    j->q = q;
    j->out = out;
    j->force_scalar = force_scalar;
    started[u] = pthread_create(&tid[u], NULL, decode_worker, j) == 0;
    if (!started[u]) decode_worker(j);
  }
  int32_t rc = RV_OK;
  for (size_t u = 0; u < units; ++u) {
    if (started[u]) pthread_join(tid[u], NULL);
    if (jobs[u].lo != jobs[u].hi && jobs[u].rc && rc == RV_OK) {
      rc = jobs[u].rc;
      if (err) *err = jobs[u].err;
    }
  }
  free(jobs);
  free(tid);
  free(started);
  return rc;
}

typedef struct scatter_job {
  const rvo_kv* kv;
  size_t layer, start, lo, hi, q_dim;
  float scale;
  const float* q;
  float* out;
  int force_scalar;
  int32_t rc;
  rv_error err;
} scatter_job;

static void* scatter_worker(void* arg) {
  scatter_job* j = arg;
  size_t n_q = j->q_dim / j->kv->head_dim;
  size_t need = rvo_scratch_len(n_q, j->kv->n_kv_heads, j->kv->head_dim, j->kv->capacity);
  float* scratch = malloc(need * 4);
  j->rc = RV_OK;
  for (size_t r = j->lo; r < j->hi; ++r) {
    j->rc = rvo_attention(j->q + r * j->q_dim, j->q_dim, j->kv, j->layer, 1, j->start + r + 1,
                          j->scale, 0, j->kv->n_kv_heads, scratch, need, j->out + r * j->q_dim,
                          j->q_dim, j->force_scalar, &j->err);
    if (j->rc) break;
  }
  free(scratch);
  return NULL;
}

/* model/prefill.rs:1322-1408: cost-balanced row shards, row r attends
 * start + r + 1 positions. */
int32_t rvo_scatter_attention(const rvo_kv* kv, size_t layer, size_t start, size_t rows,
                              size_t q_dim, float scale, const float* q, float* out,
                              size_t threads, int force_scalar, rv_error* err) {
  if (rows == 0) return RV_OK;
  size_t shards = threads ? threads : 1;
  scatter_job* jobs = calloc(shards, sizeof *jobs);
  pthread_t* tid = calloc(shards, sizeof *tid);
  int* started = calloc(shards, sizeof *started);
  for (size_t s = 0; s < shards; ++s) {
    scatter_job* j = &jobs[s];
    rvo_attention_shard_range(rows, start, shards, s, &j->lo, &j->hi);
    j->kv = kv;
    j->layer = layer;
    j->start = start;
    j->q_dim = q_dim;
    j->scale = scale;
    j->q = q;
    j->out = out;
    j->force_scalar = force_scalar;
    if (shards == 1) {
      scatter_worker(j);
      continue;
    }
    started[s] = pthread_create(&tid[s], NULL, scatter_worker, j) == 0;
    if (!started[s]) scatter_worker(j);
  }
  int32_t rc = RV_OK;
  for (size_t s = 0; s < shards; ++s) {
    if (started[s]) pthread_join(tid[s], NULL);
    if (jobs[s].rc && rc == RV_OK) {
      rc = jobs[s].rc;
      if (err) *err = jobs[s].err;
    }
  }
  free(jobs);
  free(tid);
  free(started);
  return rc;
}

/* ---- layer steps ---------------------------------------------------------- */

/* model/forward.rs:2622-2633. */
/* primitives/norm.rs:72-83: a head of `hd` values against a weight of
 * `w_len`. */
static int32_t check_norm_weight(size_t hd, size_t w_len, rv_error* err) {
  if (w_len != hd)
    return set_err(err, RV_PRIM_LENGTH_MISMATCH, hd, w_len, 0, 0, "rmsnorm_in_place: x vs weight");
  return RV_OK;
}

int32_t rvo_decode_step(rvo_kv* kv, size_t layer, float* q, size_t q_len, float* k,
                        const float* v, const float* q_norm_w, size_t q_norm_len,
                        const float* k_norm_w, size_t k_norm_len, float eps, float theta,
                        uint32_t position, float scale, float* out, size_t threads,
                        int force_scalar, rv_error* err) {
  size_t hd = kv->head_dim;
  int32_t rc;
  /* forward.rs:2622-2627: every q head, then every k head. */
  if (q_len >= hd && (rc = check_norm_weight(hd, q_norm_len, err))) return rc;
  for (size_t h = 0; h + hd <= q_len; h += hd) rvo_rmsnorm_in_place(q + h, q_norm_w, hd, eps);
  if ((rc = check_norm_weight(hd, k_norm_len, err))) return rc;
  for (size_t h = 0; h + hd <= kv->kv_dim; h += hd) rvo_rmsnorm_in_place(k + h, k_norm_w, hd, eps);
  rc = rvo_rope_neox_heads(q, q_len, q_len / hd, hd, position, theta);
  if (rc) return set_err(err, rc, hd, 0, 0, 0, "rope q");
  rc = rvo_rope_neox_heads(k, kv->kv_dim, kv->n_kv_heads, hd, position, theta);
  if (rc) return set_err(err, rc, hd, 0, 0, 0, "rope k");
  rc = rvo_kv_append(kv, layer, k, kv->kv_dim, v, kv->kv_dim, err);
  if (rc) return rc;
  return rvo_pool_decode_attention(kv, layer, scale, q, q_len, out, q_len, threads, force_scalar,
                                   err);
}

/* model/prefill.rs:2055-2111 (d) norm+rope per row at start + r, (e) append
 * every row, (f) scatter_attention. */
int32_t rvo_prefill_chunk(rvo_kv* kv, size_t layer, float* q_rows, float* k_rows,
                          const float* v_rows, size_t rows, size_t q_dim,
                          const float* q_norm_w, size_t q_norm_len, const float* k_norm_w,
                          size_t k_norm_len, float eps, float theta, size_t start, float scale,
                          float* out, size_t threads, int force_scalar, rv_error* err) {
  size_t hd = kv->head_dim, kv_dim = kv->kv_dim;
  for (size_t r = 0; r < rows; ++r) {
    uint32_t pos = (uint32_t)(start + r);
    float* q = q_rows + r * q_dim;
    float* k = k_rows + r * kv_dim;
    /* prefill.rs:2057-2076: q heads normed and rotated, then k heads. */
    int32_t rc;
    if (q_dim >= hd && (rc = check_norm_weight(hd, q_norm_len, err))) return rc;
    for (size_t h = 0; h + hd <= q_dim; h += hd) rvo_rmsnorm_in_place(q + h, q_norm_w, hd, eps);
    rc = rvo_rope_neox_heads(q, q_dim, q_dim / hd, hd, pos, theta);
    if (rc) return set_err(err, rc, hd, 0, 0, 0, "rope q");
    if ((rc = check_norm_weight(hd, k_norm_len, err))) return rc;
    for (size_t h = 0; h + hd <= kv_dim; h += hd) rvo_rmsnorm_in_place(k + h, k_norm_w, hd, eps);
    rc = rvo_rope_neox_heads(k, kv_dim, kv->n_kv_heads, hd, pos, theta);
    if (rc) return set_err(err, rc, hd, 0, 0, 0, "rope k");
  }
  for (size_t r = 0; r < rows; ++r) {
    int32_t rc = rvo_kv_append(kv, layer, k_rows + r * kv_dim, kv_dim, v_rows + r * kv_dim,
                               kv_dim, err);
    if (rc) return rc;
  }
  return rvo_scatter_attention(kv, layer, start, rows, q_dim, scale, q_rows, out, threads,
                               force_scalar, err);
}

/* model/forward.rs:2658-2705, one row: logits by dot_f32 (forward.rs:
 * 1231-1238, serial f32, each product rounded), softmax (softmax.rs:18-40),
 * top_k scans (strict >: the first index wins ties; the winner set to -inf),
 * then with norm the f32 sum of the selection in order and one division
 * each. probs is scratch of n_experts floats. */
int32_t rvo_router_topk(const float* x, size_t hidden, const float* router, size_t n_experts, size_t top_k,
                        int norm, float* probs, uint32_t* experts, float* weights) {
  if (top_k == 0 || top_k > n_experts) return RV_FWD_INVALID_TOP_K;
  if (hidden == 0) return RV_PRIM_EMPTY;
  for (size_t e = 0; e < n_experts; ++e) {
    const float* w = router + e * hidden;
    float acc = 0.0f;
    for (size_t i = 0; i < hidden; ++i) {
      const float p = w[i] * x[i];
      acc += p;
    }
    probs[e] = acc;
  }
  rvo_softmax(probs, n_experts);
  for (size_t k = 0; k < top_k; ++k) {
    size_t best_e = 0;
    float best_p = -INFINITY;
    for (size_t e = 0; e < n_experts; ++e)
      if (probs[e] > best_p) {
        best_p = probs[e];
        best_e = e;
      }
    experts[k] = (uint32_t)best_e;
    weights[k] = best_p;
    probs[best_e] = -INFINITY;
  }
  if (norm) {
    float s = 0.0f;
    for (size_t k = 0; k < top_k; ++k) s += weights[k];
    for (size_t k = 0; k < top_k; ++k) weights[k] = weights[k] / s;
  }
  return RV_OK;
}
