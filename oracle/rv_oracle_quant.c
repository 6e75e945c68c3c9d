/*
 * rv_oracle_quant.c — CPU restatement of ramvamp's quantized projections:
 * the activation quantizers, the scalar weight dequantizers and dot
 * products, and the row-range GEMV loop.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP projections and the
 * timed CPU baseline of their benchmark leg. Citations are `path:line` into
 * ramvamp's crates/core/src. Built with -ffp-contract=off -fno-fast-math
 * (oracle/Makefile): every f32 multiply and add rounds separately, as
 * Rust's do.
 *
 * The dots are the reference's scalar kernels (kernels/quants/dot.rs): the
 * integer sub-block sums are exact, each block's float contribution is
 * formed with the same operations in the same order, and the row's sum runs
 * over the blocks in order. Parity pinning lives in tests/test_oracle_quant.py.
 */
#include "rv_oracle.h"

#include <math.h>
#include <string.h>

static int32_t qerr(rv_error* err, int32_t code, uint64_t a, uint64_t b, uint64_t c, const char* what) {
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

/* ---- geometry (kernels/quants/mod.rs:60-105) ------------------------- */

size_t rvo_quant_block_weights(uint32_t format) {
  return format == RV_QF_Q8_0 ? 32 : 256;
}

size_t rvo_quant_block_bytes(uint32_t format) {
  switch (format) {
    case RV_QF_Q4_K: return 144;
    case RV_QF_Q5_K: return 176;
    case RV_QF_Q6_K: return 210;
    case RV_QF_Q8_0: return 34;
    case RV_QF_Q8_K: return 292;
    default: return 0;
  }
}

/* QuantFormat::row_bytes (mod.rs:95-105). */
int32_t rvo_quant_row_bytes(uint32_t format, size_t in_dim, size_t* row_bytes, rv_error* err) {
  if (!rvo_quant_block_bytes(format)) return qerr(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "row_bytes");
  const size_t bw = rvo_quant_block_weights(format);
  if (in_dim % bw) return qerr(err, RV_QUANT_INDIVISIBLE_ROW, format, in_dim, bw, "row_bytes");
  *row_bytes = in_dim / bw * rvo_quant_block_bytes(format);
  return RV_OK;
}

/* ---- block field helpers (kernels/quants/blocks.rs:146-176) ---------- */

static float f16_at(const uint8_t* block, size_t off) {
  return rvo_f16_to_f32((uint16_t)(block[off] | (block[off + 1] << 8)));
}

/* get_scale_min_k4 (blocks.rs:158-167). */
static void scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* ---- activation quantizers (kernels/quants/quantize.rs) -------------- */

/* quantize_row_q8_0 (quantize.rs:37-55): d = amax/127, q = round(v / d)
 * half away from zero, d stored f16-rounded. */
int32_t rvo_quantize_row_q8_0(const float* x, size_t x_len, rv_block_q8_0* out, size_t n_blocks, rv_error* err) {
  if (x_len != n_blocks * 32) return qerr(err, RV_QUANT_QUANTIZE_LEN_MISMATCH, RV_QF_Q8_0, x_len, n_blocks, "quantize");
  for (size_t b = 0; b < n_blocks; ++b) {
    const float* xs = x + 32 * b;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xs[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    out[b].d = rvo_f16_to_f32(rvo_f32_to_f16(d));
    for (int i = 0; i < 32; ++i) out[b].qs[i] = (int8_t)roundf(xs[i] * id);
  }
  return RV_OK;
}

/* quantize_row_q8_k (quantize.rs:71-106): the signed value of largest
 * magnitude (first one on ties) maps to -127; round half to even; clamp;
 * bsums per 16; d = 1/iscale in f32. */
int32_t rvo_quantize_row_q8_k(const float* x, size_t x_len, rv_block_q8_k* out, size_t n_blocks, rv_error* err) {
  if (x_len != n_blocks * 256) return qerr(err, RV_QUANT_QUANTIZE_LEN_MISMATCH, RV_QF_Q8_K, x_len, n_blocks, "quantize");
  for (size_t b = 0; b < n_blocks; ++b) {
    const float* xs = x + 256 * b;
    rv_block_q8_k* blk = &out[b];
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < 256; ++i) {
      const float av = fabsf(xs[i]);
      if (av > amax) {
        amax = av;
        max = xs[i];
      }
    }
    if (amax == 0.0f) {
      memset(blk, 0, sizeof(*blk));
      continue;
    }
    const float iscale = -127.0f / max;
    for (int i = 0; i < 256; ++i) {
      long n = lrintf(iscale * xs[i]); /* default rounding: nearest, ties to even */
      if (n < -128) n = -128;
      if (n > 127) n = 127;
      blk->qs[i] = (int8_t)n;
    }
    for (int g = 0; g < 16; ++g) {
      int32_t s = 0;
      for (int i = 0; i < 16; ++i) s += blk->qs[16 * g + i];
      blk->bsums[g] = (int16_t)s;
    }
    blk->d = 1.0f / iscale;
  }
  return RV_OK;
}

/* ---- dequantizers (kernels/quants/dequant.rs) ------------------------ */

static int32_t check_row(uint32_t format, size_t len, rv_error* err) {
  const size_t bb = rvo_quant_block_bytes(format);
  if (len % bb) return qerr(err, RV_QUANT_ROW_BYTES_NOT_BLOCK_MULTIPLE, format, len, bb, "row");
  return RV_OK;
}

/* dequantize_row_q4_k (dequant.rs:31-58) and _q5_k (:65-99). */
static void dequant_affine(const uint8_t* block, int five, float* y) {
  const float d = f16_at(block, 0), min = f16_at(block, 2);
  const uint8_t* scales = block + 4;
  const uint8_t* qh = five ? block + 16 : NULL;
  const uint8_t* qs = block + (five ? 48 : 16);
  for (int span = 0; span < 4; ++span) {
    uint8_t sc1, m1, sc2, m2;
    scale_min_k4(2 * span, scales, &sc1, &m1);
    scale_min_k4(2 * span + 1, scales, &sc2, &m2);
    const float d1 = d * (float)sc1, n1 = min * (float)m1;
    const float d2 = d * (float)sc2, n2 = min * (float)m2;
    const uint8_t* q = qs + 32 * span;
    for (int l = 0; l < 32; ++l) {
      const int hi = five && (qh[l] & (1u << (2 * span))) ? 16 : 0;
      *y++ = d1 * (float)((q[l] & 0xF) + hi) - n1;
    }
    for (int l = 0; l < 32; ++l) {
      const int hi = five && (qh[l] & (2u << (2 * span))) ? 16 : 0;
      *y++ = d2 * (float)((q[l] >> 4) + hi) - n2;
    }
  }
}

/* dequantize_row_q6_k (dequant.rs:106-134). */
static void dequant_q6k(const uint8_t* block, float* y) {
  const float d = f16_at(block, 208);
  for (int half = 0; half < 2; ++half) {
    const uint8_t* ql = block + 64 * half;
    const uint8_t* qh = block + 128 + 32 * half;
    const int8_t* sc = (const int8_t*)(block + 192 + 8 * half);
    float* yh = y + 128 * half;
    for (int l = 0; l < 32; ++l) {
      const int is = l / 16;
      const int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
      const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      yh[l] = d * (float)sc[is] * (float)q1;
      yh[l + 32] = d * (float)sc[is + 2] * (float)q2;
      yh[l + 64] = d * (float)sc[is + 4] * (float)q3;
      yh[l + 96] = d * (float)sc[is + 6] * (float)q4;
    }
  }
}

int32_t rvo_dequantize_row(uint32_t format, const uint8_t* bytes, size_t len, float* out, rv_error* err) {
  if (format == RV_QF_Q8_K || !rvo_quant_block_bytes(format))
    return qerr(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "dequantize");
  const int32_t rc = check_row(format, len, err);
  if (rc) return rc;
  const size_t bb = rvo_quant_block_bytes(format), n = len / bb;
  for (size_t b = 0; b < n; ++b) {
    const uint8_t* block = bytes + bb * b;
    switch (format) {
      case RV_QF_Q4_K: dequant_affine(block, 0, out + 256 * b); break;
      case RV_QF_Q5_K: dequant_affine(block, 1, out + 256 * b); break;
      case RV_QF_Q6_K: dequant_q6k(block, out + 256 * b); break;
      default: { /* Q8_0 (dequant.rs:140-147) */
        const float d = f16_at(block, 0);
        for (int i = 0; i < 32; ++i) out[32 * b + i] = d * (float)(int8_t)block[2 + i];
      }
    }
  }
  return RV_OK;
}

/* ---- scalar dots (kernels/quants/dot.rs) ----------------------------- */

/* weight_blocks (dot.rs:30-48). */
static int32_t dot_blocks(uint32_t format, size_t len, size_t act_blocks, rv_error* err) {
  const int32_t rc = check_row(format, len, err);
  if (rc) return rc;
  const size_t wb = len / rvo_quant_block_bytes(format);
  if (wb != act_blocks) return qerr(err, RV_QUANT_BLOCK_COUNT_MISMATCH, wb, act_blocks, 0, "dot");
  return RV_OK;
}

/* k_quant_affine_block (dot.rs:56-85): integer sums, then
 * d*sumi - dmin*sumi_mins. */
static float affine_block(const int8_t* aux, const uint8_t* scales, const rv_block_q8_k* y, float d, float dmin) {
  uint8_t sc[8], mins[8];
  for (int j = 0; j < 8; ++j) scale_min_k4(j, scales, &sc[j], &mins[j]);
  int32_t sumi_mins = 0;
  for (int g = 0; g < 16; ++g) sumi_mins += (int32_t)y->bsums[g] * (int32_t)mins[g / 2];
  int32_t sumi = 0;
  for (int j = 0; j < 8; ++j) {
    int32_t s = 0;
    for (int l = 0; l < 32; ++l) s += (int32_t)aux[32 * j + l] * (int32_t)y->qs[32 * j + l];
    sumi += (int32_t)sc[j] * s;
  }
  return d * (float)sumi - dmin * (float)sumi_mins;
}

/* vec_dot_q4_k_q8_k (dot.rs:91-112). */
static float dot_q4k(const uint8_t* row, const rv_block_q8_k* acts, size_t nb) {
  float sumf = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* block = row + 144 * b;
    const rv_block_q8_k* y = &acts[b];
    const float d = f16_at(block, 0) * y->d;
    const float dmin = f16_at(block, 2) * y->d;
    const uint8_t* qs = block + 16;
    int8_t aux[256];
    for (int span = 0; span < 4; ++span)
      for (int l = 0; l < 32; ++l) {
        aux[64 * span + l] = (int8_t)(qs[32 * span + l] & 0xF);
        aux[64 * span + 32 + l] = (int8_t)(qs[32 * span + l] >> 4);
      }
    sumf += affine_block(aux, block + 4, y, d, dmin);
  }
  return sumf;
}

/* vec_dot_q5_k_q8_k (dot.rs:118-143). */
static float dot_q5k(const uint8_t* row, const rv_block_q8_k* acts, size_t nb) {
  float sumf = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* block = row + 176 * b;
    const rv_block_q8_k* y = &acts[b];
    const float d = f16_at(block, 0) * y->d;
    const float dmin = f16_at(block, 2) * y->d;
    const uint8_t* qh = block + 16;
    const uint8_t* qs = block + 48;
    int8_t aux[256];
    for (int j = 0; j < 8; ++j) {
      const uint8_t* q = qs + 32 * (j / 2);
      const uint8_t mask = (uint8_t)(1u << j);
      for (int l = 0; l < 32; ++l) {
        const int low = j % 2 == 0 ? (q[l] & 0xF) : (q[l] >> 4);
        const int hi = (qh[l] & mask) ? 16 : 0;
        aux[32 * j + l] = (int8_t)(low + hi);
      }
    }
    sumf += affine_block(aux, block + 4, y, d, dmin);
  }
  return sumf;
}

/* vec_dot_q6_k_q8_k (dot.rs:150-179). */
static float dot_q6k(const uint8_t* row, const rv_block_q8_k* acts, size_t nb) {
  float sumf = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* block = row + 210 * b;
    const rv_block_q8_k* y = &acts[b];
    int8_t aux[256];
    for (int half = 0; half < 2; ++half) {
      const uint8_t* ql = block + 64 * half;
      const uint8_t* qh = block + 128 + 32 * half;
      int8_t* a = aux + 128 * half;
      for (int l = 0; l < 32; ++l) {
        const int h = qh[l];
        a[l] = (int8_t)(((ql[l] & 0xF) | ((h & 3) << 4)) - 32);
        a[l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32);
        a[l + 64] = (int8_t)(((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32);
        a[l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32);
      }
    }
    int32_t sumi = 0;
    for (int g = 0; g < 16; ++g) {
      const int32_t scale = (int8_t)block[192 + g];
      int32_t s = 0;
      for (int l = 0; l < 16; ++l) s += (int32_t)aux[16 * g + l] * (int32_t)y->qs[16 * g + l];
      sumi += scale * s;
    }
    sumf += f16_at(block, 208) * y->d * (float)sumi;
  }
  return sumf;
}

/* vec_dot_q8_0_q8_0 (dot.rs:185-201). */
static float dot_q80(const uint8_t* row, const rv_block_q8_0* acts, size_t nb) {
  float sumf = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* block = row + 34 * b;
    int32_t sumi = 0;
    for (int l = 0; l < 32; ++l) sumi += (int32_t)(int8_t)block[2 + l] * (int32_t)acts[b].qs[l];
    sumf += (float)sumi * (f16_at(block, 0) * acts[b].d);
  }
  return sumf;
}

int32_t rvo_vec_dot_q8_k(uint32_t format, const uint8_t* row, size_t len, const rv_block_q8_k* acts,
                         size_t n_blocks, float* out, rv_error* err) {
  if (format != RV_QF_Q4_K && format != RV_QF_Q5_K && format != RV_QF_Q6_K)
    return qerr(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "vec_dot_q8_k");
  const int32_t rc = dot_blocks(format, len, n_blocks, err);
  if (rc) return rc;
  *out = format == RV_QF_Q4_K ? dot_q4k(row, acts, n_blocks)
       : format == RV_QF_Q5_K ? dot_q5k(row, acts, n_blocks)
                              : dot_q6k(row, acts, n_blocks);
  return RV_OK;
}

int32_t rvo_vec_dot_q8_0(const uint8_t* row, size_t len, const rv_block_q8_0* acts, size_t n_blocks, float* out,
                         rv_error* err) {
  const int32_t rc = dot_blocks(RV_QF_Q8_0, len, n_blocks, err);
  if (rc) return rc;
  *out = dot_q80(row, acts, n_blocks);
  return RV_OK;
}

/* ---- GEMV (kernels/gemv.rs) ------------------------------------------ */

/* validate (gemv.rs:212-266): whole-matrix bytes, range order, range bound,
 * out length, block count, in that order. */
static int32_t gemv_validate(uint32_t format, size_t weight_len, size_t in_dim, size_t out_dim, size_t act_blocks,
                             size_t n_acts, size_t row_lo, size_t row_hi, size_t out_len, const char* what,
                             size_t* row_bytes, rv_error* err) {
  int32_t rc = rvo_quant_row_bytes(format, in_dim, row_bytes, err);
  if (rc) return rc;
  size_t expected;
  if (__builtin_mul_overflow(*row_bytes, out_dim, &expected)) expected = SIZE_MAX;  /* saturating */
  if (expected != weight_len) return qerr(err, RV_PRIM_LENGTH_MISMATCH, weight_len, expected, 0, what);
  if (row_lo > row_hi) return qerr(err, RV_PRIM_LENGTH_MISMATCH, row_lo, row_hi, 0, "gemv rows: row range start vs end");
  if (row_hi > out_dim)
    return qerr(err, RV_PRIM_LENGTH_MISMATCH, row_hi, out_dim, 0, "gemv rows: row range end vs out_dim");
  size_t wanted, wb;
  if (__builtin_mul_overflow(row_hi - row_lo, n_acts, &wanted)) wanted = SIZE_MAX;
  if (out_len != wanted) return qerr(err, RV_PRIM_LENGTH_MISMATCH, out_len, wanted, 0, what);
  if (__builtin_mul_overflow(in_dim / rvo_quant_block_weights(format), n_acts, &wb)) wb = SIZE_MAX;
  if (wb != act_blocks) return qerr(err, RV_QUANT_BLOCK_COUNT_MISMATCH, wb, act_blocks, 0, "gemv");
  return RV_OK;
}

/* gemv_q8_k_batched / gemv_q8_k_rows (gemv.rs:296-443): out[i * n_acts + a]
 * = row(row_lo + i) . act_row(a). n_acts = 1 is the single-vector form. */
int32_t rvo_gemv_q8_k(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                      const rv_block_q8_k* acts, size_t act_blocks, size_t n_acts, size_t row_lo, size_t row_hi,
                      float* out, size_t out_len, rv_error* err) {
  if (format != RV_QF_Q4_K && format != RV_QF_Q5_K && format != RV_QF_Q6_K)
    return qerr(err, RV_QUANT_UNSUPPORTED_FORMAT, format, 0, 0, "gemv_q8_k");
  size_t row_bytes;
  const int32_t rc = gemv_validate(format, weight_len, in_dim, out_dim, act_blocks, n_acts, row_lo, row_hi, out_len,
                                   "gemv_q8_k: weight bytes vs rows / out vs range", &row_bytes, err);
  if (rc) return rc;
  const size_t nb = in_dim / 256;
  for (size_t r = row_lo; r < row_hi; ++r) {
    const uint8_t* row = weight + r * row_bytes;
    for (size_t a = 0; a < n_acts; ++a) {
      const rv_block_q8_k* y = acts + a * nb;
      out[(r - row_lo) * n_acts + a] = format == RV_QF_Q4_K ? dot_q4k(row, y, nb)
                                       : format == RV_QF_Q5_K ? dot_q5k(row, y, nb)
                                                              : dot_q6k(row, y, nb);
    }
  }
  return RV_OK;
}

/* gemv_q8_0_rows / _batched (gemv.rs:544-654). */
int32_t rvo_gemv_q8_0(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                      const rv_block_q8_0* acts, size_t act_blocks, size_t n_acts, size_t row_lo, size_t row_hi,
                      float* out, size_t out_len, rv_error* err) {
  size_t row_bytes;
  const int32_t rc = gemv_validate(RV_QF_Q8_0, weight_len, in_dim, out_dim, act_blocks, n_acts, row_lo, row_hi,
                                   out_len, "gemv_q8_0: weight bytes vs rows / out vs range", &row_bytes, err);
  if (rc) return rc;
  const size_t nb = in_dim / 32;
  for (size_t r = row_lo; r < row_hi; ++r)
    for (size_t a = 0; a < n_acts; ++a)
      out[(r - row_lo) * n_acts + a] = dot_q80(weight + r * row_bytes, acts + a * nb, nb);
  return RV_OK;
}
