/*
 * ramvamp_gemv.h — C ABI of the gfx950 quantized projections either side of
 * ramvamp's attention: the activation quantizers and the k-quant / q8_0
 * GEMVs (crates/core/src/kernels/quants/{quantize,dot}.rs, kernels/gemv.rs), and the
 * per-layer attention-input and output projections that call them
 * (model/forward.rs:2574-2612, :2630-2646).
 *
 * Conventions (shared with ramvamp_attn.h):
 *  - every tensor pointer is device memory on the current HIP device, at
 *    least 4-byte aligned; RV_HOST_PTRS is refused (RV_ERR_UNSUPPORTED).
 *  - work is queued on `stream` (a hipStream_t, NULL for the null stream);
 *    RV_SYNC synchronises it before returning. Nothing here allocates.
 *  - lengths are validated on the host, in the reference's order, before
 *    any launch; on error nothing is written and the status is returned
 *    with its payload in *err (may be NULL).
 *  - results are bit-identical to the reference's scalar kernels on the same
 *    bytes: the activation integers, bsums and scales exactly, and each
 *    GEMV output because its integer sub-block sums are exact and its float
 *    operations are the scalar dot's, in the same order.
 */
#ifndef RAMVAMP_GEMV_H
#define RAMVAMP_GEMV_H

#include <stddef.h>
#include <stdint.h>

#include "ramvamp_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Formats (kernels/quants/mod.rs:60-73): block weights / bytes
 * Q4_K 256/144, Q5_K 256/176, Q6_K 256/210, Q8_0 32/34, Q8_K 256/292. */
#define RV_QF_Q4_K 1u
#define RV_QF_Q5_K 2u
#define RV_QF_Q6_K 3u
#define RV_QF_Q8_0 4u
#define RV_QF_Q8_K 5u

/* KernelError variants (kernels/error.rs); LengthMismatch is
 * RV_PRIM_LENGTH_MISMATCH with `what`, `a` left, `b` right. */
#define RV_QUANT_INDIVISIBLE_ROW 40              /* a format, b in_dim, c block_weights */
#define RV_QUANT_ROW_BYTES_NOT_BLOCK_MULTIPLE 41 /* a format, b len, c block_bytes */
#define RV_QUANT_BLOCK_COUNT_MISMATCH 42         /* a weight_blocks, b activation_blocks */
#define RV_QUANT_QUANTIZE_LEN_MISMATCH 43        /* a format, b floats, c out_blocks */
#define RV_QUANT_UNSUPPORTED_FORMAT 44           /* what, a format */

/* Activation blocks, ggml's block_q8_K / block_q8_0 field order
 * (kernels/quants/blocks.rs:178-240; the Rust structs are never serialised,
 * so this layout is the ABI's): w[j] = d * qs[j]; bsums[g] is the sum of
 * qs[16g .. 16g + 16]; Q8_0's d is the f16-rounded scale, kept as f32. */
typedef struct rv_block_q8_k {
  float d;
  int8_t qs[256];
  int16_t bsums[16];
} rv_block_q8_k; /* 292 bytes */

typedef struct rv_block_q8_0 {
  float d;
  int8_t qs[32];
} rv_block_q8_0; /* 36 bytes */

/* QuantFormat::block_weights / block_bytes (mod.rs:75-93); 0 for an
 * unknown format. */
size_t rv_quant_block_weights(uint32_t format);
size_t rv_quant_block_bytes(uint32_t format);
/* QuantFormat::row_bytes (mod.rs:95-105): RV_QUANT_INDIVISIBLE_ROW. */
int32_t rv_quant_row_bytes(uint32_t format, size_t in_dim, size_t* row_bytes, rv_error* err);

/* quantize_row_q8_0 (quantize.rs:37-55) and quantize_row_q8_k (:71-106):
 * x_len must be n_blocks * 32 (resp. 256): RV_QUANT_QUANTIZE_LEN_MISMATCH. */
int32_t rv_quantize_row_q8_0(const float* x, size_t x_len, rv_block_q8_0* out, size_t n_blocks, void* stream,
                             uint32_t flags, rv_error* err);
int32_t rv_quantize_row_q8_k(const float* x, size_t x_len, rv_block_q8_k* out, size_t n_blocks, void* stream,
                             uint32_t flags, rv_error* err);

/* gemv_q8_k_rows (gemv.rs:386-411): out[i] = weight_row(row_lo + i) . acts
 * for the k-quant formats (Q4_K, Q5_K, Q6_K; others
 * RV_QUANT_UNSUPPORTED_FORMAT). `weight` is the whole row-major matrix
 * (weight_len = out_dim * row_bytes(in_dim)); acts holds in_dim/256 blocks;
 * out_len = row_hi - row_lo. gemv_q8_k (:347-368) is the range 0..out_dim. */
int32_t rv_gemv_q8_k_rows(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                          const rv_block_q8_k* acts, size_t act_blocks, size_t row_lo, size_t row_hi, float* out,
                          size_t out_len, void* stream, uint32_t flags, rv_error* err);
int32_t rv_gemv_q8_k(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                     const rv_block_q8_k* acts, size_t act_blocks, float* out, size_t out_len, void* stream,
                     uint32_t flags, rv_error* err);
/* gemv_q8_0_rows / gemv_q8_0 (gemv.rs:544-615): Q8_0 weights against Q8_0
 * activations (in_dim/32 blocks). */
int32_t rv_gemv_q8_0_rows(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                          const rv_block_q8_0* acts, size_t act_blocks, size_t row_lo, size_t row_hi, float* out,
                          size_t out_len, void* stream, uint32_t flags, rv_error* err);
int32_t rv_gemv_q8_0(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                     const rv_block_q8_0* acts, size_t act_blocks, float* out, size_t out_len, void* stream,
                     uint32_t flags, rv_error* err);

/* gemv.rs:444-478 `gemv_q8_k_batched` and :616-651 `gemv_q8_0_batched`:
 * out[i * n_acts + a] = row(row_lo + i) . act_row(a) for i < row_hi - row_lo
 * and a < n_acts, where `acts` holds n_acts rows of in_dim / 256 Q8_K (or
 * in_dim / 32 Q8_0) blocks, act_blocks in all. Validation as the single-row
 * forms with out_len = (row_hi - row_lo) * n_acts and act_blocks =
 * n_acts * in_dim / block_weights (saturating). Every output is
 * bit-identical to the single-row GEMV of that activation row: the integer
 * sums run on int8 MFMA tiles (exact), the float operations are the scalar
 * dot's in block order. */
int32_t rv_gemv_q8_k_batched(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim,
                             size_t out_dim, const rv_block_q8_k* acts, size_t act_blocks, size_t n_acts,
                             size_t row_lo, size_t row_hi, float* out, size_t out_len, void* stream, uint32_t flags,
                             rv_error* err);
int32_t rv_gemv_q8_0_batched(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                             const rv_block_q8_0* acts, size_t act_blocks, size_t n_acts, size_t row_lo,
                             size_t row_hi, float* out, size_t out_len, void* stream, uint32_t flags, rv_error* err);

/* A prefill chunk's attention projections (model/prefill.rs:1985-2053 and
 * :2113-2154), rows row-major. rv_attn_in_proj_rows quantizes each normed
 * row [n_rows][hidden] to Q8_K and Q8_0 (into scratch), then writes
 * q_rows[n_rows][q_dim], k_rows[n_rows][kv_dim] and v_rows[n_rows][kv_dim]
 * with the batched GEMVs (the reference's transposes are the store layout);
 * rv_attn_out_proj_rows quantizes attn_rows[n_rows][q_dim] to Q8_K and adds
 * Wo . row into residual_rows[n_rows][hidden] (residual + o, one f32 add per
 * element). Each projected value equals the single-row GEMV of its row. */
size_t rv_attn_in_proj_rows_scratch_bytes(size_t n_rows, size_t hidden);
int32_t rv_attn_in_proj_rows(const float* normed_rows, size_t n_rows, size_t hidden, uint32_t q_format,
                             const uint8_t* wq, size_t wq_len, float* q_rows, size_t q_dim, const uint8_t* wk,
                             size_t wk_len, float* k_rows, size_t kv_dim, uint32_t v_format, const uint8_t* wv,
                             size_t wv_len, float* v_rows, void* scratch, size_t scratch_len, void* stream,
                             uint32_t flags, rv_error* err);
size_t rv_attn_out_proj_rows_scratch_bytes(size_t n_rows, size_t q_dim);
int32_t rv_attn_out_proj_rows(const float* attn_rows, size_t n_rows, size_t q_dim, uint32_t o_format,
                              const uint8_t* wo, size_t wo_len, float* residual_rows, size_t hidden, void* scratch,
                              size_t scratch_len, void* stream, uint32_t flags, rv_error* err);

/* One layer's attention-input projections (forward.rs:2574-2612): the
 * normed hidden row is quantized to Q8_K and Q8_0 into `scratch`, then
 * q = Wq . x (q_format k-quant, q_dim rows), k = Wk . x (Q8_0, kv_dim rows)
 * and v = Wv . x (v_format k-quant, kv_dim rows) run as one launch. Each
 * output equals rv_gemv_* on the same quantized row. scratch_len must be at
 * least rv_attn_in_proj_scratch_bytes(hidden) (RV_PRIM_LENGTH_MISMATCH). */
size_t rv_attn_in_proj_scratch_bytes(size_t hidden);
int32_t rv_attn_in_proj(const float* normed, size_t hidden, uint32_t q_format, const uint8_t* wq, size_t wq_len,
                        float* q, size_t q_dim, const uint8_t* wk, size_t wk_len, float* k, size_t kv_dim,
                        uint32_t v_format, const uint8_t* wv, size_t wv_len, float* v, void* scratch,
                        size_t scratch_len, void* stream, uint32_t flags, rv_error* err);
/* The output projection (forward.rs:2630-2646): attn_out quantized to Q8_K
 * into `scratch`, then o = Wo . a (o_format k-quant, `hidden` rows of q_dim
 * weights). scratch_len >= rv_attn_out_proj_scratch_bytes(q_dim). */
size_t rv_attn_out_proj_scratch_bytes(size_t q_dim);
int32_t rv_attn_out_proj(const float* attn_out, size_t q_dim, uint32_t o_format, const uint8_t* wo, size_t wo_len,
                         float* o, size_t hidden, void* scratch, size_t scratch_len, void* stream, uint32_t flags,
                         rv_error* err);

#ifdef __cplusplus
}
#endif

#endif /* RAMVAMP_GEMV_H */
