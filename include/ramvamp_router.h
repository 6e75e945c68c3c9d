/*
 * ramvamp_router.h — C ABI of the MoE router's decision on gfx950
 * (model/forward.rs:2658-2705): per row, logits = the router matrix times
 * the normed row (dot_f32, forward.rs:1231-1238: one serial f32 sum per
 * expert), softmax over all experts (primitives/softmax.rs:18-40), the
 * top_k largest probabilities in descending order (first index wins ties),
 * renormalized to sum 1 when norm_topk_prob.
 *
 * Conventions of ramvamp_gemv.h: device pointers (4-byte aligned),
 * RV_HOST_PTRS refused, work on `stream`, RV_SYNC waits. Every value equals
 * the reference's: the dots keep the serial order and separate multiply and
 * add, the softmax's exponentials are f64 (sum in expert order), the
 * selection and the renormalization are the reference's loops.
 */
#ifndef RAMVAMP_ROUTER_H
#define RAMVAMP_ROUTER_H

#include <stddef.h>
#include <stdint.h>

#include "ramvamp_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* forward.rs:229-237 ForwardError::InvalidTopK: a top_k, b n_experts. */
#define RV_FWD_INVALID_TOP_K 48

/* x: n_rows rows of `hidden` normed values; router: n_experts rows of
 * `hidden` f32 weights; outputs n_rows x top_k expert indices and weights.
 * Errors: RV_FWD_INVALID_TOP_K (top_k 0 or above n_experts, checked first),
 * RV_PRIM_EMPTY (hidden 0: no row), RV_PRIM_LENGTH_MISMATCH (router_len !=
 * n_experts * hidden). n_experts <= 1024, hidden <= 16384. */
int32_t rv_router_topk(const float* x, size_t n_rows, size_t hidden, const float* router, size_t router_len,
                       size_t n_experts, size_t top_k, int norm_topk_prob, uint32_t* experts, float* weights,
                       void* stream, uint32_t flags, rv_error* err);

#ifdef __cplusplus
}
#endif

#endif /* RAMVAMP_ROUTER_H */
