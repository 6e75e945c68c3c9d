// rv_internal.hpp — host-side state of a device KV cache and the kernel
// launchers the C ABI (rv_abi.cpp) drives. Not part of the public ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "../../include/ramvamp_attn.h"

struct rv_kv {
  size_t n_layers = 0, n_kv_heads = 0, head_dim = 0, capacity = 0, kv_dim = 0, plane = 0;
  int elem = RV_ELEM_F16;
  int device = 0;
  void* k = nullptr;  // [n_layers][capacity][kv_dim], elem-sized, device
  void* v = nullptr;
  std::vector<size_t> lens;  // per-layer cursors (kv/mod.rs:147), host-side
  hipStream_t stream = nullptr;

  // Device workspace, grown on first need and then reused by every call:
  // decode and prefill split partials, normalised q rows / RoPE tables.
  void* ws = nullptr;
  size_t ws_bytes = 0;
  float* qbuf = nullptr;  // normalised + rotated q rows of the fused steps
  size_t qbuf_bytes = 0;
  // Buffers a grown workspace, qbuf, staging or staged copy replaced: kept
  // until rv_kv_free, since a graph captured earlier may still address them.
  std::vector<void*> retired;
  size_t retired_bytes = 0;
  void retire(void* p, size_t bytes) {
    retired.push_back(p);
    retired_bytes += bytes;
  }
  // The XCD split merge's tickets, zero between calls (each call's last
  // arriver resets its own): 9 * n_kv_heads counters, one per 128-byte line;
  // then the device status words (rv_kv_device_status).
  unsigned* tickets = nullptr;
  // Recorded on the old stream when rv_kv_set_stream moves the cache to a
  // new one, which then waits for it.
  hipEvent_t order_ev = nullptr;
  // Prefill's staged copy of each layer's K/V tiles (MFMA type and LDS
  // layout), kept across calls so a reused prefix is converted once:
  // positions [0, staged_pos[layer]) are current for staged_mode[layer].
  // Every write below a layer's staged_pos (truncate, clear) lowers it;
  // appends land at or above it.
  std::vector<void*> staged;
  std::vector<size_t> staged_bytes, staged_pos;
  std::vector<uint32_t> staged_mode;
  // The F16 / BF16 prefill's split-fold tickets: one 128-byte line per
  // (kv head, 256-vector block) unit, zero between calls.
  unsigned* pf_tickets = nullptr;
  size_t pf_ticket_units = 0;
  // Staging for RV_HOST_PTRS calls.
  void* stage = nullptr;
  size_t stage_bytes = 0;
  // The device-position decode step's (cos, sin) table: for positions
  // [0, rope_n), 64 cos then 64 sin (f64 on the host, cast to f32, as the
  // host-position step computes them) at rope_theta; grown, never freed
  // while the cache lives (a captured token graph addresses it).
  float* rope_tab = nullptr;
  size_t rope_n = 0;
  float rope_theta = 0.f;

  int64_t tune_decode_split_len = 0;
  int64_t tune_prefill_kv_split = 0;
  int64_t tune_decode_waves = 0;
  int64_t tune_prefill_rows = 0;
  int64_t tune_decode_hg = 0;
  int64_t tune_decode_impl = 0;  // 0 auto (MFMA tiles: head_dim 128, group <= 16), 1 VALU subgroups, 3 LDS-staged tiles
  int64_t tune_decode_depth = 0;  // tiles in flight per wave (1, 2, 4); 0 auto
  int64_t tune_decode_merge = 0;  // 0 auto, 1 in-launch XCD merge, 2 separate merge kernel
  // The dispatcher deals a launch's workgroups to the XCDs round robin on this
  // device (checked at rv_kv_new): the XCD merge may rely on it.
  bool xcd_ok = false;

  // RV_TUNE_KERNEL_TIMING: event pairs around the dominant kernel of each
  // call, folded into timed_ms / timed_n when read (or when the pool fills).
  bool timing = false;
  std::vector<hipEvent_t> ev;
  size_t ev_used = 0;
  double timed_ms = 0;
  uint64_t timed_n = 0;

  size_t elem_size() const { return elem == RV_ELEM_F32 ? 4 : 2; }
  char* k_layer(size_t layer) const { return (char*)k + layer * plane * elem_size(); }
  char* v_layer(size_t layer) const { return (char*)v + layer * plane * elem_size(); }
};

namespace rv {

// Layout of rv_kv::tickets (see there). The XCD merge's counters sit one per
// 128-byte line (atomics on one line serialize): (XCD slot, kv head) at line
// slot * n_kv_heads + head, level 2 at line 8 * n_kv_heads + head.
inline size_t xcd_ticket_pad(const rv_kv* kv) { return kv->n_kv_heads; }
inline size_t xcd_ticket_off(const rv_kv*) { return 0; }
inline size_t status_off(const rv_kv* kv) { return 9 * 32 * kv->n_kv_heads; }
inline size_t ticket_words(const rv_kv* kv) { return status_off(kv) + 32; }
inline unsigned* xcd_tickets(const rv_kv* kv) { return kv->tickets ? kv->tickets + xcd_ticket_off(kv) : nullptr; }
inline unsigned* dev_status(const rv_kv* kv) { return kv->tickets ? kv->tickets + status_off(kv) : nullptr; }
// Whether the workgroups of a launch whose indices agree mod 8 run on one XCD
// on `device` (a probe, once per device; the device must be current).
bool xcd_dealing_ok(int device);

// Result of a launch helper: hipSuccess or the first failing HIP call.
struct HipStatus {
  hipError_t e = hipSuccess;
  const char* what = nullptr;
};

// Compute units of the MI355X, which the launch plans balance work over.
constexpr long kCUs = 256;

// Workspace of at least `bytes` on the cache's device. When it must grow it
// is allocated at max(bytes, bound) (callers pass the most any call of the
// same geometry can ask for at the cache's capacity, so a decode loop never
// grows it), and the old buffer is retired, not freed. Growth under graph
// capture is refused with hipErrorStreamCaptureUnsupported.
HipStatus ensure_workspace(rv_kv* kv, size_t bytes, size_t bound = 0);
// Whether work on s is being captured into a graph.
bool capturing(hipStream_t s);
// The normalised-q buffer, with the workspace's growth rules.
HipStatus ensure_qbuf(rv_kv* kv, size_t bytes);
// RV_ERR_UNSUPPORTED for a call that would have to allocate under graph
// capture, RV_ERR_HIP for any other HIP failure.
inline int32_t status_code(hipError_t e) {
  return e == hipErrorStreamCaptureUnsupported ? RV_ERR_UNSUPPORTED : RV_ERR_HIP;
}

// RV_TUNE_KERNEL_TIMING: the event pair the next dominant-kernel launch
// records its own start and end into (hipExtLaunchKernelGGL), or two nulls
// when timing is off or the stream is being captured.
struct TimedPair {
  hipEvent_t start = nullptr, stop = nullptr;
};
TimedPair timing_pair(rv_kv* kv, hipStream_t s);
// Adds every recorded pair to timed_ms / timed_n (waits for the last one).
void timing_fold(rv_kv* kv);

// Launch that fills `tp` with the kernel's start and end when it is set.
template <typename F, typename... Args>
inline void launch_timed(const TimedPair& tp, F kernel, dim3 grid, dim3 block, hipStream_t s, Args... args) {
  if (tp.start)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, tp.start, tp.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}

// True when the MFMA prefill kernel covers this geometry and extent (else the
// ABI runs each row through the decode kernel with its own position limit).
bool prefill_supported(const rv_kv* kv, size_t group, size_t positions);

// ---- prologue / append (rv_prologue.hip) ------------------------------------
// RoPE inverse frequencies theta^(-2i/d) for i < d/2, computed on the host in
// f64 (primitives/rope.rs:35-36) and passed by value.
constexpr int kMaxHalf = 256;
struct InvFreq {
  double f[kMaxHalf];
};
void fill_inv_freq(InvFreq& t, size_t head_dim, float theta);

// Append `rows` rows (kv_dim each) of k and v, as given, at cursor `pos0` of
// `layer`.
HipStatus launch_append(const rv_kv* kv, size_t layer, size_t pos0, const float* k, const float* v, size_t rows,
                        hipStream_t s);
// A layer's staged K/V tiles (prefill's MFMA-typed copy) that a row
// prologue also writes its k and v rows into; base == nullptr: none.
struct StageDst {
  char* base = nullptr;
  int tile_stride = 0;  // tiles between consecutive kv heads
  uint32_t mode = 0;    // RV_PREFILL_EXACT / F16 / BF16
};
// Rows of (q, k, v) at RoPE positions pos0 + r: q heads RMSNormed with q_w
// and rotated into q_out (rows x n_q x head_dim; n_q may be 0), k heads
// RMSNormed with k_w and rotated into the cache at cache_row + r, v heads
// copied there. With rope_tab, each row's (cos, sin) as f32 are also written
// there (per row head_dim/2 cos, then head_dim/2 sin), for a fused q
// prologue downstream.
// With sd (head_dim 128 only), the k and v rows as the cache holds them are
// also written into the staged tiles at cache_row + r, and the rest of the
// last tile is zeroed.
// With qp (and sd, so the chunk's q heads run in the same launch), q heads
// go into the prepared layout of the F16 / BF16 prefill instead of q_out.
struct QPrep {
  char* base = nullptr;
  int group = 0;       // query heads per kv head
  int qr = 0;          // rows per unit: its columns / group
  int n_rb = 0;        // units per kv head
  float qscale = 0.f;  // log2(e) * softmax scale
  int vectors = 0;     // columns per unit (64 or 128)
  // The cache's (cos, sin) table by position (ensure_rope_tab), read instead
  // of each wave computing its row's angles in f64.
  const float* rope = nullptr;
};
// Bytes of the prepared queries of a chunk of `rows` rows, and their layout,
// for units of `vectors` columns (prefill_vectors).
size_t qprep_bytes(size_t rows, size_t n_kv_heads, size_t group, int vectors);
QPrep qprep_plan(char* base, size_t rows, size_t group, float scale, int vectors);
// Columns per unit of the F16 / BF16 prefill kernel for a chunk of `rows`
// rows at `start` (64 or 128; the prepared queries are laid out for it).
int prefill_vectors(const rv_kv* kv, size_t rows, size_t start, size_t group);
HipStatus launch_row_prologue(const rv_kv* kv, size_t layer, size_t cache_row, const float* q, float* q_out,
                              size_t n_q, const float* k, const float* v, size_t rows, const float* q_w,
                              const float* k_w, float eps, const InvFreq& inv, size_t pos0, float* rope_tab,
                              const StageDst* sd, hipStream_t s, const QPrep* qp = nullptr);

// ---- decode (rv_decode.hip) ------------------------------------------------------
// The workspace the MFMA decode path can need for any call on this cache
// (whole kv range, groups up to 16, up to its capacity) with the default
// launch shape; 0 when the geometry takes another path. rv_kv_new reserves
// it, so a decode call can be captured into a graph without a warm-up call.
size_t decode_ws_bound(const rv_kv* kv);
// out[(h - kv_lo*group)*d + i] for the kv-head range [kv_lo, kv_hi), all
// `positions` of `layer`. q is the full post-RoPE query.
// A caller's workspace, used instead of the cache's (nothing is allocated,
// no timing events are made); the launch fails if it is too small.
struct Workspace {
  void* base;
  size_t bytes;
};
HipStatus launch_decode(rv_kv* kv, const float* q, size_t n_q_heads, size_t layer, size_t positions,
                        float scale, size_t kv_lo, size_t kv_hi, float* out, hipStream_t s,
                        const Workspace* ws = nullptr);
// Workspace bytes launch_decode needs for this call's geometry.
size_t decode_ws_need(const rv_kv* kv, size_t n_q_heads, size_t positions, size_t n_heads);
// rv_decode_attention_noalloc's device scratch: kNoAllocScratchBytes in a
// file-scope device array (rv_decode.hip); its address on `device` (which
// must be current), resolved once per device.
constexpr size_t kNoAllocScratchBytes = RV_NOALLOC_SCRATCH_BYTES;
HipStatus noalloc_scratch(int device, void** ptr);

// The decode step's prologue carried into the tile kernel (forward.rs:
// 2617-2633): q pre-norm (each workgroup normalizes and rotates its group's
// heads as it loads them), and the token's pre-norm k and v rows, which the
// workgroup of the split holding position positions - 1 writes into that
// cache row (k normalized and rotated) before its tiles read it. (cos, sin)
// of the token's position for pair i, computed on the host in f64.
// With d_pos (a token graph's step, replayed for every token), the token's
// position is read from device memory instead: positions = min(*d_pos,
// max_pos) + 1, the launch planned for max_pos + 1 positions (splits past
// the token write empty partials), and (cos, sin) read from tab (the
// cache's rope_tab: 64 cos then 64 sin per position).
struct DecodePro {
  const float* k;
  const float* v;
  const float* q_w;
  const float* k_w;
  float eps;
  float cs[64], sn[64];
  const uint32_t* d_pos = nullptr;
  const float* tab = nullptr;
  int max_pos = 0;
  // With d_pos: a position above max_pos is refused (no row written, out
  // untouched) and recorded here: [0] RV_KV_CAPACITY_EXCEEDED, [1] layer,
  // [2] the position, [3] max_pos + 1 (the first refusal since the last read).
  uint32_t* status = nullptr;
  uint32_t layer = 0;
};
// True when launch_decode_pro covers the geometry (head_dim 128, group <= 16:
// the MFMA tile kernel); the caller then skips the row prologue.
bool decode_pro_supported(const rv_kv* kv, size_t n_q_heads);
// *d_position += n on s (a kernel, so a captured graph can carry it).
HipStatus launch_position_advance(uint32_t* d_position, uint32_t n, hipStream_t s);
// The whole decode step over positions (the token's row is positions - 1).
HipStatus launch_decode_pro(rv_kv* kv, const float* q_raw, size_t n_q_heads, size_t layer, size_t positions,
                            float scale, const DecodePro& pro, float* out, hipStream_t s);

// ---- prefill (rv_prefill.hip) -------------------------------------------------
// The q prologue fused into the prefill kernels' query loads: RMSNorm with
// w and eps, rotation with the rows' (cos, sin) table (from
// launch_row_prologue, or the cache's rope_tab): row r's at tab + r * 128,
// 64 cos then 64 sin.
// With `prepped` (F16 / BF16 only), the queries are already normed, rotated,
// scaled and rounded in the prepared layout (QPrep) and w, eps, tab and the
// q rows are not read.
struct QNorm {
  const float* w = nullptr;
  float eps = 0.f;
  const float* tab = nullptr;
  const char* prepped = nullptr;
};
// Before a prefill chunk appends `rows` rows at pos0 = len(layer) and runs
// launch_prefill: readies the layer's persistent staged copy in `mode`
// (stages the rows the prefix gained since it was last current, up to pos0)
// and marks [0, pos0 + rows) current, so that the chunk's row prologue
// writes its own rows there (sd) and launch_prefill stages nothing. Under
// graph capture sd->base stays null: a captured call stages into the
// workspace instead.
HipStatus prepare_prefill_stage(rv_kv* kv, size_t layer, size_t pos0, size_t rows, uint32_t mode,
                                hipStream_t s, StageDst* sd);
// Row r of q_rows (rows x q_dim) attends positions 0..start+r+1; q_rows are
// post-RoPE, or the raw projections when qn is given.
HipStatus launch_prefill(rv_kv* kv, const float* q_rows, size_t rows, size_t n_q_heads, size_t layer,
                         size_t start, float scale, float* out, uint32_t mode, const QNorm* qn, hipStream_t s);

// The F16 / BF16 prefill's fold tickets for `units` units (not under capture).
HipStatus ensure_prefill_tickets(rv_kv* kv, size_t units);

// The largest staged copy one layer's prefill can hold (EXACT tiles over the
// whole capacity).
size_t prefill_stage_bound(const rv_kv* kv);

// rv_decode_step's validation alone (no launch), for callers that validate
// a whole composite call before launching any of it.
int32_t decode_step_check(const rv_kv* kv, size_t layer, size_t q_len, size_t position, size_t q_norm_len,
                          size_t k_norm_len, rv_error* err);
// rv_prefill_chunk's validation alone.
int32_t prefill_chunk_check(const rv_kv* kv, size_t layer, size_t rows, size_t q_dim, size_t start,
                            size_t q_norm_len, size_t k_norm_len, rv_error* err);
// rv_decode_step_dev's validation alone.
int32_t decode_step_dev_check(const rv_kv* kv, size_t layer, size_t q_len, size_t max_position, size_t q_norm_len,
                              size_t k_norm_len, rv_error* err);
// The device-position step's (cos, sin) table covering positions [0, n).
HipStatus ensure_rope_tab(rv_kv* kv, float theta, size_t n);

}  // namespace rv
