/*
 * ramvamp_block.h — C ABI of one layer's attention block for one token on
 * gfx950, the device-resident form of model/forward.rs:2570-2650:
 *
 *   normed   = rmsnorm(residual, attn_norm, eps)          (:2572)
 *   q, k, v  = Wq, Wk, Wv . quantize(normed)              (:2574-2612)
 *   q, k     = per-head QK-RMSNorm, then NeoX RoPE at `position` (:2617-2629)
 *   append k, v at the layer's cursor; attn_out = attention(q) over the layer (:2631-2633)
 *   residual += Wo . quantize_q8_k(attn_out)              (:2636-2650)
 *
 * It replaces that sequence of host calls (and the host round trips of q, k,
 * v and attn_out between them) with four launches on the cache's stream:
 * the input projections with the RMSNorm fused into each workgroup's
 * activation quantization, the attention (its query heads normalized and
 * rotated as they load, the token's k and v rows normalized, rotated and
 * appended by the workgroup of the last split) and its split merge, and the
 * output projection with the residual add fused into its stores. Captured into one graph per token, the 48
 * layers' blocks replay with no host work between them.
 *
 * Conventions are those of ramvamp_attn.h and ramvamp_gemv.h: device
 * pointers only (4-byte aligned; RV_HOST_PTRS is refused), RV_SYNC waits for
 * the cache's stream, every check runs before any launch in the reference's
 * order, and on error nothing is written (`residual` and the cache stay as
 * they were). The projections are bit-identical to the reference's scalar
 * kernels given the normalized row; the normalization, prologue and attention
 * follow the reference's arithmetic within the tolerances of those paths.
 */
#ifndef RAMVAMP_BLOCK_H
#define RAMVAMP_BLOCK_H

#include <stddef.h>
#include <stdint.h>

#include "ramvamp_attn.h"
#include "ramvamp_gemv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One layer's attention weights (model/weights: attn_norm, attn_q, attn_k,
 * attn_v, attn_q_norm, attn_k_norm, attn_output), device pointers. */
typedef struct rv_attn_block_weights {
  const float* attn_norm;  /* [hidden] */
  uint32_t q_format;       /* RV_QF_Q4_K / Q5_K / Q6_K */
  const uint8_t* wq;       /* q_dim rows of `hidden` weights */
  size_t wq_len;
  const uint8_t* wk;       /* Q8_0, kv_dim rows of `hidden` weights */
  size_t wk_len;
  uint32_t v_format;       /* RV_QF_Q4_K / Q5_K / Q6_K */
  const uint8_t* wv;       /* kv_dim rows of `hidden` weights */
  size_t wv_len;
  const float* q_norm;     /* [head_dim] */
  const float* k_norm;     /* [head_dim] */
  uint32_t o_format;       /* RV_QF_Q4_K / Q5_K / Q6_K */
  const uint8_t* wo;       /* hidden rows of `q_dim` weights */
  size_t wo_len;
  size_t q_norm_len;       /* head_dim, checked as rv_decode_step checks it */
  size_t k_norm_len;
} rv_attn_block_weights;

/* Bytes of device scratch rv_attn_block_decode needs: q, k, v and attn_out,
 * plus, for rows wider than 8192, the normalized and quantized rows. */
size_t rv_attn_block_scratch_bytes(size_t hidden, size_t q_dim, size_t kv_dim);

/* forward.rs:2570-2650 for `layer`: residual[hidden] is read and updated in
 * place; q_dim = n_q_heads * head_dim; the token's k and v rows land at the
 * layer's cursor, which advances by one; q and k rotate at `position`
 * (normally the cursor). Validation order: the rmsnorm (RV_PRIM_EMPTY for
 * hidden 0), the input projections as rv_attn_in_proj, the decode step as
 * rv_decode_step, the output projection as rv_attn_out_proj, then scratch,
 * flags and pointers. */
int32_t rv_attn_block_decode(rv_kv* kv, size_t layer, float* residual, size_t hidden, size_t q_dim,
                             const rv_attn_block_weights* w, float eps, float theta, size_t position,
                             float scale, void* scratch, size_t scratch_len, uint32_t flags, rv_error* err);

/* No counterpart in the reference: rv_attn_block_decode with the decode step
 * as rv_decode_step_dev (the token's position read from *d_position when the
 * step runs, planned for max_position; the layer's host cursor does not move,
 * rv_kv_commit adds the rows), for a token graph captured once and replayed
 * per token. A null d_position is RV_ERR_NULL_ARG. */
int32_t rv_attn_block_decode_dev(rv_kv* kv, size_t layer, float* residual, size_t hidden, size_t q_dim,
                                 const rv_attn_block_weights* w, float eps, float theta,
                                 const uint32_t* d_position, size_t max_position, float scale, void* scratch,
                                 size_t scratch_len, uint32_t flags, rv_error* err);

/* The same block for a prefill chunk of n_rows tokens at positions start ..
 * start + n_rows - 1 (model/prefill.rs:1975-2154, the attention half of a
 * layer): each residual row normalized (rmsnorm_rows), quantized both ways,
 * the batched q/k/v projections (rv_attn_in_proj_rows), the chunk's QK norm,
 * RoPE, append and causal attention (rv_prefill_chunk; flags carries its
 * RV_PREFILL_* mode), and the batched output projection added into each
 * residual row (rv_attn_out_proj_rows). residual_rows[n_rows][hidden] is
 * updated in place; start must equal the layer's length. Launches: the row
 * norm, two quantizers, three batched GEMVs, the prefill chunk's, one
 * quantizer and one batched GEMV. */
size_t rv_attn_block_prefill_scratch_bytes(size_t n_rows, size_t hidden, size_t q_dim, size_t kv_dim);
int32_t rv_attn_block_prefill(rv_kv* kv, size_t layer, float* residual_rows, size_t n_rows, size_t hidden,
                              size_t q_dim, const rv_attn_block_weights* w, float eps, float theta, size_t start,
                              float scale, void* scratch, size_t scratch_len, uint32_t flags, rv_error* err);

#ifdef __cplusplus
}
#endif

#endif /* RAMVAMP_BLOCK_H */
