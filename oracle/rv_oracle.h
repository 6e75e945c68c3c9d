/*
 * rv_oracle.h — CPU restatement of ramvamp's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP path is
 * compared against, and the timed CPU baseline of the benchmark. Nothing in
 * the product (ramvamp_amd/, include/) links, loads or calls it.
 *
 * Every function follows a reference function line by line, cited as
 * `path:line` into ramvamp's crates/core/src. Build flags matter: the
 * reference (Rust) never contracts a*b+c into an FMA, so this file is built
 * with -ffp-contract=off -fno-fast-math (oracle/Makefile).
 *
 * Error codes and the payload struct are the product's (include/ramvamp_attn.h)
 * so a test can compare a GPU call's failure with the oracle's directly.
 */
#ifndef RV_ORACLE_H
#define RV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/ramvamp_attn.h"
#include "../include/ramvamp_gemv.h"
#include "../include/ramvamp_router.h"

#ifdef __cplusplus
extern "C" {
#endif

/* kernels/quants/f16.rs:17-32 and :39-91. */
float rvo_f16_to_f32(uint16_t bits);
uint16_t rvo_f32_to_f16(float x);
/* Bulk forms (for tests). */
void rvo_f16_to_f32_n(const uint16_t* src, float* dst, size_t n);
void rvo_f32_to_f16_n(const float* src, uint16_t* dst, size_t n);

/* kv/mod.rs:132-148: linear planes [n_layers][capacity][kv_dim], per-layer
 * cursors. `elem` RV_ELEM_F16 stores f16 bits (the reference's format),
 * RV_ELEM_F32 stores f32 with the same indexing. */
typedef struct rvo_kv {
  size_t n_layers, n_kv_heads, head_dim, capacity, kv_dim, plane;
  int elem;
  void* k;
  void* v;
  size_t* lens;
} rvo_kv;

int32_t rvo_kv_projected_bytes(size_t n_layers, size_t n_kv_heads, size_t head_dim,
                               size_t capacity, int elem, uint64_t* bytes, rv_error* err);
int32_t rvo_kv_new(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity,
                   int elem, rvo_kv** out, rv_error* err);
void rvo_kv_free(rvo_kv* kv);
int32_t rvo_kv_len(const rvo_kv* kv, size_t layer, size_t* len, rv_error* err);
int rvo_kv_is_empty(const rvo_kv* kv);
int32_t rvo_kv_seq_len(const rvo_kv* kv, size_t* len, rv_error* err);
int32_t rvo_kv_append(rvo_kv* kv, size_t layer, const float* k, size_t k_len, const float* v,
                      size_t v_len, rv_error* err);
void rvo_kv_clear(rvo_kv* kv);
int32_t rvo_kv_truncate(rvo_kv* kv, size_t new_len, rv_error* err);
/* kv/mod.rs:428-441: copies kv_dim elements of the plane's type into dst. */
int32_t rvo_kv_read_row(const rvo_kv* kv, int plane_v, size_t layer, size_t pos, void* dst,
                        rv_error* err);

/* primitives/softmax.rs:18-40 (in place; RV_PRIM_LENGTH_MISMATCH on empty). */
int32_t rvo_softmax(float* x, size_t n);
/* primitives/norm.rs:72-90. */
int32_t rvo_rmsnorm_in_place(float* x, const float* w, size_t n, float eps);
/* primitives/rope.rs:82-105. */
int32_t rvo_rope_neox_heads(float* x, size_t x_len, size_t n_heads, size_t head_dim,
                            uint32_t position, float theta);

/* attention.rs:337-353. */
size_t rvo_scratch_len(size_t n_q_heads, size_t n_kv_heads, size_t head_dim,
                       size_t max_positions);

/* attention.rs:426-859, all twelve entry points in one: `has_limit` picks
 * attention_at (positions = limit) over decode_attention; [kv_lo, kv_hi) is
 * the kv-head range (0..n_kv_heads for the whole-vector forms); `scratch` /
 * `scratch_len` is the borrowed carve (`_in` forms) or NULL for the owning
 * form (sized from capacity, attention.rs:993-1020); `force_scalar` pins the
 * scalar body instead of the AVX2+F16C one (attention.rs:141-145). */
int32_t rvo_attention(const float* q, size_t q_len, const rvo_kv* kv, size_t layer,
                      int has_limit, size_t limit, float scale, size_t kv_lo, size_t kv_hi,
                      float* scratch, size_t scratch_len, float* out, size_t out_len,
                      int force_scalar, rv_error* err);

/* True when the AVX2+F16C body covers head_dim (attention.rs:198-209). */
int rvo_avx2_path_covers(size_t head_dim);

/* model/forward.rs:2052-2063 `kv_head_range`. */
void rvo_kv_head_range(size_t n_kv_heads, size_t units, size_t slot_lo, size_t slot_hi,
                       size_t* lo, size_t* hi);
/* model/prefill.rs:1211-1281 `attention_cost` / `attention_shard_range`. */
void rvo_attention_shard_range(size_t rows, size_t start, size_t shards, size_t index,
                               size_t* lo, size_t* hi);

/* model/forward.rs:1914-2031 `pool_decode_attention` over `threads` OS
 * threads (the pool's shards), serial below 8 positions. */
int32_t rvo_pool_decode_attention(const rvo_kv* kv, size_t layer, float scale, const float* q,
                                  size_t q_len, float* out, size_t out_len, size_t threads,
                                  int force_scalar, rv_error* err);
/* model/prefill.rs:1322-1408 `scatter_attention` over `threads` threads. */
int32_t rvo_scatter_attention(const rvo_kv* kv, size_t layer, size_t start, size_t rows,
                              size_t q_dim, float scale, const float* q, float* out,
                              size_t threads, int force_scalar, rv_error* err);

/* model/forward.rs:2622-2633: q/k per-head RMSNorm, RoPE, append, attention.
 * q (q_len) and k (kv_dim) are modified in place, as in the reference. */
int32_t rvo_decode_step(rvo_kv* kv, size_t layer, float* q, size_t q_len, float* k,
                        const float* v, const float* q_norm_w, size_t q_norm_len,
                        const float* k_norm_w, size_t k_norm_len, float eps, float theta,
                        uint32_t position, float scale, float* out, size_t threads,
                        int force_scalar, rv_error* err);
/* model/prefill.rs:2055-2111 steps (d)-(f); q_rows/k_rows modified in place. */
int32_t rvo_prefill_chunk(rvo_kv* kv, size_t layer, float* q_rows, float* k_rows,
                          const float* v_rows, size_t rows, size_t q_dim,
                          const float* q_norm_w, size_t q_norm_len, const float* k_norm_w,
                          size_t k_norm_len, float eps, float theta, size_t start, float scale,
                          float* out, size_t threads, int force_scalar, rv_error* err);

/* Per-row prologue alone (for tests): norm + rope of `n_heads` heads. */
int32_t rvo_norm_rope_heads(float* x, size_t n_heads, size_t head_dim, const float* w,
                            float eps, float theta, uint32_t position);

/* ---- quantized projections (rv_oracle_quant.c) ---- */
/* QuantFormat geometry (kernels/quants/mod.rs:75-105). */
size_t rvo_quant_block_weights(uint32_t format);
size_t rvo_quant_block_bytes(uint32_t format);
int32_t rvo_quant_row_bytes(uint32_t format, size_t in_dim, size_t* row_bytes, rv_error* err);
/* quantize.rs:37-55 and :71-106. */
int32_t rvo_quantize_row_q8_0(const float* x, size_t x_len, rv_block_q8_0* out, size_t n_blocks, rv_error* err);
int32_t rvo_quantize_row_q8_k(const float* x, size_t x_len, rv_block_q8_k* out, size_t n_blocks, rv_error* err);
/* dequant.rs: Q4_K, Q5_K, Q6_K and Q8_0 rows (len bytes) into out. */
int32_t rvo_dequantize_row(uint32_t format, const uint8_t* bytes, size_t len, float* out, rv_error* err);
/* dot.rs scalar dots: one weight row of `len` bytes against n_blocks
 * activation blocks. */
int32_t rvo_vec_dot_q8_k(uint32_t format, const uint8_t* row, size_t len, const rv_block_q8_k* acts,
                         size_t n_blocks, float* out, rv_error* err);
int32_t rvo_vec_dot_q8_0(const uint8_t* row, size_t len, const rv_block_q8_0* acts, size_t n_blocks, float* out,
                         rv_error* err);
/* gemv.rs row-range GEMVs against n_acts activation rows
 * (out[i * n_acts + a]; n_acts = 1: gemv_*_rows). */
int32_t rvo_gemv_q8_k(uint32_t format, const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                      const rv_block_q8_k* acts, size_t act_blocks, size_t n_acts, size_t row_lo, size_t row_hi,
                      float* out, size_t out_len, rv_error* err);
int32_t rvo_gemv_q8_0(const uint8_t* weight, size_t weight_len, size_t in_dim, size_t out_dim,
                      const rv_block_q8_0* acts, size_t act_blocks, size_t n_acts, size_t row_lo, size_t row_hi,
                      float* out, size_t out_len, rv_error* err);

/* model/forward.rs:2658-2705: one row's router decision (probs: n_experts floats of scratch). */
int32_t rvo_router_topk(const float* x, size_t hidden, const float* router, size_t n_experts, size_t top_k,
                        int norm, float* probs, uint32_t* experts, float* weights);

#ifdef __cplusplus
}
#endif

#endif /* RV_ORACLE_H */
