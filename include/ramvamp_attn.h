/*
 * ramvamp_attn.h — C ABI of the MI355X (gfx950) GQA attention hot path.
 *
 * This is the drop-in boundary for ramvamp's per-layer attention. Every
 * entry point below replaces one reference interface, cited as
 * `path:line` into the ramvamp tree (crates/core/src/...). The library is
 * `libramvamp_attn.so`, built with hipcc for gfx950 only.
 *
 * Conventions
 *  - Every call returns an `int32_t` status: RV_OK (0) or one of the codes
 *    below. When `err` is non-NULL it receives the status plus the payload
 *    fields of the reference error variant (field meaning per code below).
 *  - Validation runs on the host, in the reference's precedence, before any
 *    device work is queued, so `out` is untouched on every error.
 *  - Tensor pointers (q, k, v, out, norm weights) are device pointers on the
 *    cache's device unless `flags` carries RV_HOST_PTRS, in which case they
 *    are host pointers and the call copies in, computes and copies out
 *    before it returns.
 *  - With device pointers the call is asynchronous on the cache's stream
 *    (rv_kv_set_stream; default: the null stream). Calls on one cache are
 *    serialised by that stream and share its device workspace: one cache
 *    per host thread, never two streams on one cache at once.
 *  - Sizes and indices are `size_t`, element counts (not bytes) unless named
 *    `*_bytes`.
 */
#ifndef RAMVAMP_ATTN_H
#define RAMVAMP_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RV_ABI_VERSION 1u

/* ---- status codes ------------------------------------------------------
 * KvError variants (crates/core/src/kv/mod.rs:39-123). Payload: a..d.  */
#define RV_OK 0
#define RV_KV_INVALID_DIMS 1          /* a n_layers, b n_kv_heads, c head_dim, d capacity, what reason */
#define RV_KV_LAYER_OUT_OF_RANGE 2    /* a layer, b n_layers */
#define RV_KV_ROW_LEN_MISMATCH 3      /* what "k"|"v", a got, b expected */
#define RV_KV_CAPACITY_EXCEEDED 4     /* a layer, b capacity */
#define RV_KV_POSITION_OUT_OF_RANGE 5 /* a layer, b pos, c len */
#define RV_KV_RAGGED_LAYERS 6         /* a shortest, b longest */
#define RV_KV_TRUNCATE_BEYOND_LENGTH 7 /* a requested, b len */
/* AttentionError variants (crates/core/src/kernels/attention.rs:218-311). A
 * KvError raised inside attention keeps its KV code (the reference wraps it
 * as AttentionError::Kv, which is transparent). */
#define RV_ATTN_Q_LEN_INDIVISIBLE 16  /* a q_len, b head_dim */
#define RV_ATTN_GQA_GROUP_MISMATCH 17 /* a n_q_heads, b n_kv_heads */
#define RV_ATTN_OUT_LEN_MISMATCH 18   /* a out_len, b expected */
#define RV_ATTN_EMPTY_LAYER 19        /* a layer */
#define RV_ATTN_KV_HEAD_RANGE 20      /* a start, b end, c n_kv_heads */
#define RV_ATTN_SCRATCH_TOO_SHORT 21  /* a len, b need */
/* Primitive errors of the fused prologue (kernels/primitives/error.rs). */
#define RV_PRIM_INVALID_HEAD_DIM 24   /* a head_dim (rope needs it even, nonzero) */
#define RV_PRIM_LENGTH_MISMATCH 25    /* what, a left, b right */
#define RV_PRIM_EMPTY 26              /* what (an empty row to normalize) */
/* Errors of this library with no reference counterpart. */
#define RV_ERR_NULL_ARG 32            /* what argument */
#define RV_ERR_UNSUPPORTED 33         /* what, a value */
#define RV_ERR_HIP 34                 /* what call, a hipError_t */
#define RV_ERR_BAD_ELEM 35            /* a elem */

typedef struct rv_error {
  int32_t code;
  uint64_t a, b, c, d;
  const char* what; /* static string, never freed */
} rv_error;

/* Element type of the cache planes. RV_ELEM_F16 is the reference's own
 * format (f16 bits, round-to-nearest-even on append, kv/mod.rs:336-368);
 * RV_ELEM_F32 keeps the identical [layer][capacity][kv_dim] indexing with
 * 4-byte elements. */
typedef enum rv_elem { RV_ELEM_F16 = 1, RV_ELEM_F32 = 2 } rv_elem;

/* flags */
#define RV_HOST_PTRS 0x1u   /* tensor pointers are host memory */
#define RV_SYNC 0x2u        /* synchronise the cache's stream before returning */
/* Prefill arithmetic (rv_attention_at_rows / rv_prefill_chunk only; decode is
 * always fp32 arithmetic). Default (0) = RV_PREFILL_EXACT. EXACT and F16 take
 * their operands (q, K, V, and P <= 2^8) through f16: values must stay below
 * 65504 in magnitude, and EXACT keeps its ~2^-21 relative products only for
 * values above f16's normal minimum (2^-14); BF16 has fp32's range. */
#define RV_PREFILL_EXACT 0x00u /* split-f16 MFMA, fp32-equivalent products */
#define RV_PREFILL_F16 0x10u   /* single-pass f16 MFMA inputs, fp32 accumulate */
#define RV_PREFILL_BF16 0x20u  /* single-pass bf16 MFMA inputs, fp32 accumulate */
#define RV_PREFILL_MODE_MASK 0x30u

/* Opaque device-resident KV cache: K and V planes on one GPU, per-layer
 * cursors on the host, one HIP stream, the decode/prefill workspace. */
typedef struct rv_kv rv_kv;

uint32_t rv_abi_version(void);
/* Static, human-readable name of a status code ("RV_OK", ...). */
const char* rv_status_name(int32_t code);

/* attention.rs:337-353 `scratch_len`: the f32 scratch a reference CPU call
 * needs, `(n_q_heads / n_kv_heads) * max_positions + 2 * head_dim`,
 * saturating, division-safe. The device path keeps its own workspace; the
 * `_in` entry points below still take the caller's scratch length and
 * report RV_ATTN_SCRATCH_TOO_SHORT exactly where the reference does. */
size_t rv_scratch_len(size_t n_q_heads, size_t n_kv_heads, size_t head_dim,
                      size_t max_positions);

/* ---- KV cache (crates/core/src/kv/mod.rs) ---------------------------- */

/* kv/mod.rs:237-259 `KvCache::projected_bytes`, for either element type
 * (2 planes * n_layers * capacity * n_kv_heads * head_dim * elem size). */
int32_t rv_kv_projected_bytes(size_t n_layers, size_t n_kv_heads, size_t head_dim,
                              size_t capacity, rv_elem elem, uint64_t* bytes,
                              rv_error* err);

/* kv/mod.rs:163-181 `KvCache::new`: zeroed planes on `device`, every cursor 0. */
int32_t rv_kv_new(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity,
                  rv_elem elem, int device, rv_kv** out, rv_error* err);
void rv_kv_free(rv_kv* kv);
/* Stream every later call on this cache is queued on (a hipStream_t). */
int32_t rv_kv_set_stream(rv_kv* kv, void* hip_stream, rv_error* err);
int32_t rv_kv_synchronize(rv_kv* kv, rv_error* err);

/* kv/mod.rs:262-287 accessors. */
size_t rv_kv_n_layers(const rv_kv* kv);
size_t rv_kv_n_kv_heads(const rv_kv* kv);
size_t rv_kv_head_dim(const rv_kv* kv);
size_t rv_kv_capacity(const rv_kv* kv);
size_t rv_kv_kv_dim(const rv_kv* kv);
int32_t rv_kv_elem(const rv_kv* kv);
/* kv/mod.rs:291 `len`, :297 `is_empty`, :312 `seq_len`. */
int32_t rv_kv_len(const rv_kv* kv, size_t layer, size_t* len, rv_error* err);
int rv_kv_is_empty(const rv_kv* kv);
int32_t rv_kv_seq_len(const rv_kv* kv, size_t* len, rv_error* err);

/* kv/mod.rs:336-368 `append`: one row of `n_kv_heads * head_dim` f32 for
 * each of K and V, converted to the plane's element type (f16: RNE). */
int32_t rv_kv_append(rv_kv* kv, size_t layer, const float* k, size_t k_len,
                     const float* v, size_t v_len, uint32_t flags, rv_error* err);
/* `rows` appends in one call: the loop at model/prefill.rs:2081-2087.
 * k and v hold `rows * kv_dim` f32. All-or-nothing: capacity is checked for
 * the whole chunk first (RV_KV_CAPACITY_EXCEEDED reports the layer). */
int32_t rv_kv_append_rows(rv_kv* kv, size_t layer, const float* k, const float* v,
                          size_t rows, size_t row_len, uint32_t flags, rv_error* err);
/* kv/mod.rs:383-385 `clear` and :410-420 `truncate`. */
void rv_kv_clear(rv_kv* kv);
int32_t rv_kv_truncate(rv_kv* kv, size_t new_len, rv_error* err);
/* kv/mod.rs:449-460 `k_layer` / `v_layer`: the device address of a layer's
 * plane and the element count the view covers (`len(layer) * kv_dim`). */
int32_t rv_kv_k_layer(const rv_kv* kv, size_t layer, const void** dev, size_t* n_elems,
                      rv_error* err);
int32_t rv_kv_v_layer(const rv_kv* kv, size_t layer, const void** dev, size_t* n_elems,
                      rv_error* err);
/* kv/mod.rs:428-441 `k_row` / `v_row`, copied to host memory: `dst` gets
 * kv_dim elements of the plane's type (u16 f16 bits or f32). */
int32_t rv_kv_read_row(const rv_kv* kv, int plane_v, size_t layer, size_t pos, void* dst,
                       rv_error* err);

/* ---- attention (crates/core/src/kernels/attention.rs) ---------------- */

/* attention.rs:426 `decode_attention`: q is the full post-RoPE query
 * (`n_q_heads * head_dim` f32), out the same length, every position the
 * layer holds. Precedence (attention.rs:926-989): q length, GQA grouping,
 * layer, positions, kv range, out length. */
int32_t rv_decode_attention(const rv_kv* kv, const float* q, size_t q_len, size_t layer,
                            float scale, float* out, size_t out_len, uint32_t flags,
                            rv_error* err);
/* attention.rs:484 `decode_attention_in`: also checks the caller's scratch
 * length against rv_scratch_len, after `out`. */
int32_t rv_decode_attention_in(const rv_kv* kv, const float* q, size_t q_len, size_t layer,
                               float scale, size_t scratch_len, float* out, size_t out_len,
                               uint32_t flags, rv_error* err);
/* attention.rs:586 `decode_attention_kv_range_in`: kv heads [kv_lo, kv_hi);
 * q is the full vector, out the range's own `(kv_hi-kv_lo)*group*head_dim`
 * buffer from index 0. An empty in-range request is a validated no-op. */
int32_t rv_decode_attention_kv_range_in(const rv_kv* kv, const float* q, size_t q_len,
                                        size_t layer, float scale, size_t kv_lo, size_t kv_hi,
                                        size_t scratch_len, float* out, size_t out_len,
                                        uint32_t flags, rv_error* err);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). rv_decode_attention with device pointers only, whose
 * split partials (or scores, on the generic path) live in a fixed
 * file-scope device array of RV_NOALLOC_SCRATCH_BYTES that each GPU holds
 * until the process ends, instead of the cache's workspace; it allocates
 * nothing and makes no timing events. Same validation and results (bit for
 * bit) as rv_decode_attention. RV_HOST_PTRS, or a call whose scratch need
 * exceeds the array, is RV_ERR_UNSUPPORTED (a = bytes needed, b = the
 * limit; a = 0 for host pointers). Every call on one GPU shares the array:
 * calls that overlap on one GPU (other streams, other caches) race. */
#define RV_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int32_t rv_decode_attention_noalloc(const rv_kv* kv, const float* q, size_t q_len, size_t layer,
                                    float scale, float* out, size_t out_len, uint32_t flags,
                                    rv_error* err);

/* attention.rs:666 `attention_at`: positions 0..positions only (the causal
 * limit is a length). positions == 0 -> RV_ATTN_EMPTY_LAYER; positions
 * past len(layer) -> RV_KV_POSITION_OUT_OF_RANGE. */
int32_t rv_attention_at(const rv_kv* kv, const float* q, size_t q_len, size_t layer,
                        size_t positions, float scale, float* out, size_t out_len,
                        uint32_t flags, rv_error* err);
/* attention.rs:732 `attention_at_in`. */
int32_t rv_attention_at_in(const rv_kv* kv, const float* q, size_t q_len, size_t layer,
                           size_t positions, float scale, size_t scratch_len, float* out,
                           size_t out_len, uint32_t flags, rv_error* err);
/* attention.rs:807 `attention_at_kv_range_in`. */
int32_t rv_attention_at_kv_range_in(const rv_kv* kv, const float* q, size_t q_len,
                                    size_t layer, size_t positions, float scale, size_t kv_lo,
                                    size_t kv_hi, size_t scratch_len, float* out,
                                    size_t out_len, uint32_t flags, rv_error* err);

/* model/prefill.rs:1322-1408 `scatter_attention`: `rows` query rows of
 * q_dim f32 each; row r attends positions 0..start+r+1 (prefill.rs:1394).
 * One call replaces the pool fan-out. Each row is validated as the
 * reference's per-row attention_at_in would be, in row order, before any
 * launch; the first failing row's error is returned and out is untouched
 * (the reference may leave earlier rows written, prefill.rs:1310-1320).
 * flags selects the MFMA arithmetic (RV_PREFILL_*). */
int32_t rv_attention_at_rows(const rv_kv* kv, const float* q_rows, size_t rows, size_t q_dim,
                             size_t layer, size_t start, float scale, float* out,
                             uint32_t flags, rv_error* err);

/* ---- fused layer steps ------------------------------------------------ */

/* model/forward.rs:2622-2633, one decode token of one layer: per-head
 * RMSNorm of q (n_q_heads heads) and k (n_kv_heads heads) with the shared
 * [head_dim] weights and `eps` (primitives/norm.rs:18-90), NeoX RoPE of both
 * at `position` with base `theta` (primitives/rope.rs:31-105), KvCache::append
 * of (k, v), then decode attention over every position of the layer.
 * q/k/v are pre-norm; q_len = n_q_heads*head_dim, k_len = v_len = kv_dim.
 * A norm weight whose length is not head_dim is RV_PRIM_LENGTH_MISMATCH
 * (a = head_dim, b = its length), as rmsnorm_in_place reports it
 * (primitives/norm.rs:72-83): q's weight first, then k's. */
int32_t rv_decode_step(rv_kv* kv, size_t layer, const float* q, size_t q_len, const float* k,
                       size_t k_len, const float* v, size_t v_len, const float* q_norm_w,
                       size_t q_norm_len, const float* k_norm_w, size_t k_norm_len, float eps,
                       float theta, size_t position, float scale, float* out, size_t out_len,
                       uint32_t flags, rv_error* err);

/* ---- token graph (no counterpart in the reference) ---------------------
 * For callers that capture one token's layer steps into a HIP graph once and
 * replay it for every token (the per-token decode loop of forward.rs:2568-2650
 * without a host round trip per step). rv_decode_step with the token's
 * position read from device memory (*d_position, a uint32) when the step
 * runs: the row lands at position *d_position of the layer and q and k rotate
 * at that position, so the cache is expected to hold exactly *d_position rows
 * then (the reference's decode keeps position == len). The launch is planned
 * for max_position + 1 positions (workgroups past the token's position find
 * nothing to do and contribute nothing). max_position >= capacity is
 * RV_KV_CAPACITY_EXCEEDED. A step that finds *d_position (as an unsigned
 * value) above max_position writes no cache row and leaves `out` untouched,
 * and records RV_KV_CAPACITY_EXCEEDED in the cache's device status, which
 * rv_kv_device_status and rv_kv_commit report (the device form of append's
 * refusal when a layer is full, kv/mod.rs:352-357). The host cursor does not
 * move: rv_kv_commit adds the rows the replays wrote.
 * The first call for a (theta, max_position) builds the (cos, sin) table and
 * workspace and must not be captured; later calls may be. Device pointers
 * only (RV_HOST_PTRS is RV_ERR_UNSUPPORTED); head_dim 128 and a group of at
 * most 16 (else RV_ERR_UNSUPPORTED). Results equal rv_decode_step's within
 * fp32 reassociation (the splits follow max_position, not the length). */
int32_t rv_decode_step_dev(rv_kv* kv, size_t layer, const float* q, size_t q_len, const float* k,
                           size_t k_len, const float* v, size_t v_len, const float* q_norm_w,
                           size_t q_norm_len, const float* k_norm_w, size_t k_norm_len, float eps,
                           float theta, const uint32_t* d_position, size_t max_position, float scale,
                           float* out, size_t out_len, uint32_t flags, rv_error* err);
/* Adds `rows` to the layer's length (the rows device-position steps wrote);
 * past the capacity is RV_KV_CAPACITY_EXCEEDED and nothing changes. It first
 * synchronises the cache's stream and reports a device status left by a
 * refused step exactly as rv_kv_device_status does (nothing changes then
 * either). */
int32_t rv_kv_commit(rv_kv* kv, size_t layer, size_t rows, rv_error* err);
/* No reference counterpart (the reference has no device-side steps). Waits
 * for the cache's stream, then returns the status a device-position step
 * recorded since the last read and clears it: RV_OK, or
 * RV_KV_CAPACITY_EXCEEDED with a = the first refused layer, b = the
 * positions that step was planned for (its max_position + 1, the capacity it
 * was given), c = the position it read. */
int32_t rv_kv_device_status(rv_kv* kv, rv_error* err);
/* Queues *d_position += n on the cache's stream (a token graph's last node). */
int32_t rv_position_advance(rv_kv* kv, uint32_t* d_position, uint32_t n, rv_error* err);

/* model/prefill.rs:2055-2111 steps (d)-(f) for one layer of a chunk: the
 * same prologue per row at absolute position start+r, the whole chunk's
 * K/V appended, then causal attention where row r sees start+r+1 positions.
 * `start` must equal len(layer) (the chunk continues the cache). The norm
 * weights' lengths are checked as rv_decode_step's (when rows > 0). */
int32_t rv_prefill_chunk(rv_kv* kv, size_t layer, const float* q_rows, const float* k_rows,
                         const float* v_rows, size_t rows, size_t q_dim, const float* q_norm_w,
                         size_t q_norm_len, const float* k_norm_w, size_t k_norm_len, float eps,
                         float theta, size_t start, float scale, float* out, uint32_t flags,
                         rv_error* err);

/* Tuning knobs of the decode/prefill launches (0 = built-in heuristic).
 * Exposed for benchmarking sweeps; results never depend on them beyond
 * floating-point reassociation within the stated tolerance. */
#define RV_TUNE_DECODE_SPLIT_LEN 1 /* positions per decode split (rounded to the workgroup step) */
#define RV_TUNE_PREFILL_KV_SPLIT 2 /* KV splits per prefill block of query vectors (1..8) */
#define RV_TUNE_DECODE_WAVES 3     /* waves per MFMA decode workgroup: 4 (default) or 8; VALU path: 4 or 8 (default) */
#define RV_TUNE_PREFILL_ROWS 4     /* EXACT prefill: query rows per workgroup, 8 or 16 (group 8) */
#define RV_TUNE_DECODE_HG 5        /* query heads per VALU decode workgroup: 1, 2, 4 or 8 */
#define RV_TUNE_DECODE_IMPL 6      /* decode kernel: 0 auto (MFMA tiles when head_dim 128 and group <= 16; f16 planes on f16
                                      MFMA operands split hi/lo), 1 VALU subgroups, 2 MFMA tiles with fp32 operands,
                                      3 MFMA tiles staged through LDS (4-wave workgroups) */
#define RV_TUNE_KERNEL_TIMING 7    /* 1: time the dominant kernel of every call with HIP events (not under capture) */
#define RV_TUNE_DECODE_DEPTH 9     /* 16-position tiles in flight per decode wave: 1 (default), 2 or 4 (f16 planes) */
#define RV_TUNE_DECODE_MERGE 11    /* decode split merge: 0 auto, 1 inside the tile launch (a first level inside each
                                      XCD's L2, then across XCDs), 2 a second kernel */
int32_t rv_kv_set_tuning(rv_kv* kv, int32_t knob, int64_t value, rv_error* err);

/* No reference counterpart: benchmark instrumentation. With
 * RV_TUNE_KERNEL_TIMING on, every decode/prefill call that is not being
 * captured into a graph launches its dominant kernel (the tile/split decode
 * kernel, the prefill kernel) with a pair of HIP events that record that
 * kernel's own start and end on the cache's stream (hipExtLaunchKernelGGL).
 * This synchronises the stream, returns the summed event time in
 * milliseconds and the number of timed launches since the last read, and
 * resets both. */
int32_t rv_kv_kernel_time(rv_kv* kv, double* total_ms, uint64_t* launches, rv_error* err);

/* No reference counterpart: the device memory this cache holds, in bytes.
 * rv_kv_projected_bytes is the reference's planes-only budget
 * (kv/mod.rs:237-259: 2 * n_layers * capacity * kv_dim * element size);
 * this adds what the device path keeps beside the planes. *now is what is
 * allocated at the call (planes, workspace including buffers a growth
 * retired, normalised-q buffer, host-pointer staging, the (cos, sin) table,
 * tickets and status, and every layer's prefill staged copy made so far);
 * *bound is that total once every layer holds a staged copy sized for its
 * capacity in the costliest prefill mode (EXACT tiles: 17/16 of the layer's
 * f32 planes or 17/8 of its f16 planes; F16/BF16 tiles take half the f32
 * planes or all of the f16 planes) and
 * the table covers the capacity; growth past it comes only from a prefill
 * chunk or RV_HOST_PTRS call larger than any before. Either may be null. */
int32_t rv_kv_device_bytes(rv_kv* kv, uint64_t* now, uint64_t* bound, rv_error* err);
/* No reference counterpart: rv_kv_device_bytes' *bound for a cache of this
 * geometry before any call has grown it, computed from the geometry alone
 * (no device needed): rv_kv_projected_bytes' planes, the decode workspace
 * rv_kv_new reserves (at least 1 MiB), the merge tickets and status words,
 * an EXACT staged copy per layer over its capacity (head_dim 128; none
 * otherwise) and the (cos, sin) table over the capacity
 * (capacity * head_dim * 4 bytes). Errors as rv_kv_projected_bytes. */
int32_t rv_kv_projected_device_bytes(size_t n_layers, size_t n_kv_heads, size_t head_dim, size_t capacity,
                                     rv_elem elem, uint64_t* bytes, rv_error* err);

/* No reference counterpart: diagnostics. *ok = 1 when the cache's device
 * deals the workgroups of a launch to its XCDs round robin (checked by a
 * probe when the cache was made), which the in-launch XCD merge of the
 * decode splits relies on; 0 otherwise (the decode then merges in a second
 * launch). */
int32_t rv_kv_xcd_dealing(rv_kv* kv, int32_t* ok, rv_error* err);

#ifdef __cplusplus
}
#endif

#endif /* RAMVAMP_ATTN_H */
