// rv_prefill.hip — causal chunked-prefill attention on gfx950 MFMA.
//
// Replaces scatter_attention -> attention_at_in per row
// (crates/core/src/model/prefill.rs:1322-1408 -> kernels/attention.rs:732):
// query row r of the chunk attends cache positions 0..start+r+1.
//
// Two kernels per call (plus a merge when the KV axis is split):
//
// 1. prefill_stage_kernel converts the layer's K and V rows [0, positions)
//    once into the MFMA element type (f16 / bf16, or for the split mode
//    hi + lo f16 with each K row and each V column of a tile scaled by its
//    power of two) and lays each 64-position tile out exactly as the attention
//    kernel wants it in LDS: K row-major, V transposed with its positions
//    permuted into the order the S^T accumulator produces P, both with their
//    16-byte chunks XOR-swizzled so the MFMA operand reads are free of bank
//    conflicts. Every row block of the chunk then re-reads this compact copy
//    (half the bytes of an fp32 cache) instead of converting on the fly.
//
// 2. The attention kernel: one workgroup per (kv head, block of query
//    vectors, KV split). Its query vectors are every q head of the GQA group
//    for each of its rows, so each staged K/V tile feeds all heads. Tiles
//    stream into LDS with direct-to-LDS loads (global_load_lds_dwordx4: no
//    registers, no conversion), issued from inline assembly so the compiler
//    adds no wait for them before LDS reads. Per tile:
//      S^T[t][m] = sum_d K[t][d] Q[m][d]      (A = K from LDS, B = Q in registers)
//      O^T[d][m] += sum_t V[t][d] P[m][t]     (A = V^T from LDS, B = P in registers)
//    Computing S transposed puts a query vector's scores in the lanes that
//    hold it as the B operand P^T needs, so P never leaves registers. Both
//    kernels are software-pipelined inside each wave: a tile's softmax work
//    runs between the MFMAs of its neighbours.
//    prefill_kernel (EXACT) works on v_mfma_f32_16x16x32_f16, 16 or 32
//    columns per wave; prefill32_kernel (F16 / BF16) on
//    v_mfma_f32_32x32x16_{f16,bf16}, 32 columns per wave.
//
// Arithmetic modes (flags RV_PREFILL_*):
//   EXACT, the fp32 parity mode, for any finite fp32 operands: each K row,
//          each V column of a tile and each q vector scaled by a power of
//          two that puts its largest magnitude in [2^13, 2^14), split as hi
//          + lo f16; products hi*hi + lo*hi + hi*lo in fp32 (~2^-21 of the
//          row and vector maxima), the scales undone exactly on the fp32
//          scores and on each tile's O^T rows; P (< 2^8) as f16 hi + lo,
//          three products per PV term.
//   F16 / BF16: one MFMA per product, fp32 accumulate.
// Softmax is online in fp32 (exp2, log2(e) folded into the score scale), with
// the running maximum moved only when a tile exceeds it by 2^8.
//
// KV splits (short chunks, too few row blocks to fill the chip): each split
// writes partial (O, max, sum) columns; EXACT folds them with an fp32
// log-sum-exp in a further launch (prefill_merge_kernel), F16 / BF16 in the
// same launch (the last split of a unit to finish, on the splits' XCD).
#include "rv_device.hpp"
#include "rv_internal.hpp"
#include "rv_staged.hpp"

#include <algorithm>
#include <type_traits>

namespace rv {
namespace {

constexpr int kWG = 256;
constexpr int kD = 128;
constexpr int kMaxKvSplits = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegSentinel = -1.0e30f;

// Stage kernel: one workgroup per (kv head, tile in [tile_lo, tile_lo +
// n_tiles), plane K or V); a kv head's tiles are tile_stride apart. Rows at
// or past `positions` are staged as zeros. Loads are whole rows per wave
// instruction (fp32: thread i reads row 8j + i/32, elements 4(i%32)..+3 for
// j < 8; f16: row 16j + i/16, elements 8(i%16)..+7 for j < 4), all issued
// before any is used. K goes straight to its swizzled rows; V is transposed
// through LDS.
template <typename T>
struct StageLoad;
template <>
struct StageLoad<float> {
  static constexpr int kN = 8, kE = 4;
  f32x4 x[8];
  __device__ static int row(int j, int tid) { return 8 * j + tid / 32; }
  __device__ static int col(int tid) { return 4 * (tid % 32); }
  __device__ void load(const float* __restrict__ base, int kv_dim, int t0, int positions, int tid) {
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      const int t = t0 + row(j, tid);
      x[j] = t < positions ? *reinterpret_cast<const f32x4*>(base + (size_t)t * kv_dim + col(tid))
                           : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __device__ float get(int j, int e) const { return x[j][e]; }
};
template <>
struct StageLoad<_Float16> {
  static constexpr int kN = 4, kE = 8;
  f16x8 x[4];
  __device__ static int row(int j, int tid) { return 16 * j + tid / 16; }
  __device__ static int col(int tid) { return 8 * (tid % 16); }
  __device__ void load(const _Float16* __restrict__ base, int kv_dim, int t0, int positions, int tid) {
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      const int t = t0 + row(j, tid);
      x[j] = t < positions ? *reinterpret_cast<const f16x8*>(base + (size_t)t * kv_dim + col(tid)) : f16x8{};
    }
  }
  __device__ float get(int j, int e) const { return (float)x[j][e]; }
};

template <int MODE, typename T>
__global__ __launch_bounds__(kWG) void prefill_stage_kernel(const T* __restrict__ kl, const T* __restrict__ vl,
                                                            int kv_dim, int positions, int tile_stride, int tile_lo,
                                                            int n_tiles, char* __restrict__ stage) {
  typedef typename Op<MODE>::E E;
  typedef typename Op<MODE>::V8 V8;
  typedef E EN __attribute__((ext_vector_type(StageLoad<T>::kE)));
  constexpr bool kSplit = Op<MODE>::kSplit;
  constexpr int P = kSplit ? 2 : 1;
  constexpr int NE = StageLoad<T>::kE;
  const int plane = blockIdx.x & 1;
  const int tile = tile_lo + (int)(blockIdx.x >> 1) % n_tiles, kvh = (int)(blockIdx.x >> 1) / n_tiles;
  const int tid = threadIdx.x;
  char* dst = stage + ((size_t)kvh * tile_stride + tile) * kTileBytes<MODE>;
  const int t0 = tile * kBT;
  StageLoad<T> ld;
  ld.load((plane ? vl : kl) + (size_t)kvh * kD, kv_dim, t0, positions, tid);
  if (plane == 0) {
    // NE elements = a half (fp32) or a whole (f16) 16-byte chunk of row r,
    // whose kD / NE threads are adjacent lanes; the split mode scales the row
    // by its exponent e (from their max over the row) and records 2^-e.
    const int c = StageLoad<T>::col(tid);
#pragma unroll
    for (int j = 0; j < StageLoad<T>::kN; ++j) {
      const int r = StageLoad<T>::row(j, tid);
      int ex = 0;
      if constexpr (kSplit) {
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < NE; ++e) amax = fmaxf(amax, fabsf(ld.get(j, e)));
#pragma unroll
        for (int w = 1; w < kD / NE; w <<= 1) amax = fmaxf(amax, __shfl_xor(amax, w, 64));
        ex = scale_exponent(amax);
        if (c == 0) *reinterpret_cast<float*>(dst + kScaleOffset + 4 * r) = ldexpf(1.0f, -ex);
      }
      EN hi, lo;
#pragma unroll
      for (int e = 0; e < NE; ++e) split2v<E>(kSplit ? ldexpf(ld.get(j, e), ex) : ld.get(j, e), hi, lo, e);
      const int off = k_off(r, c / 8) + 2 * (c % 8);
      *reinterpret_cast<EN*>(dst + off) = hi;
      if constexpr (P == 2) *reinterpret_cast<EN*>(dst + kPlaneBytes + off) = lo;
    }
    return;
  }
  __shared__ float vt[kBT][kD + 1];
#pragma unroll
  for (int j = 0; j < StageLoad<T>::kN; ++j)
#pragma unroll
    for (int e = 0; e < NE; ++e) vt[StageLoad<T>::row(j, tid)][StageLoad<T>::col(tid) + e] = ld.get(j, e);
  __syncthreads();
  // Thread -> V^T row d = tid / 2, chunks 4 (tid % 2) .. +3. The split mode
  // scales the tile's column d by its exponent c (from the column's max over
  // the tile, both threads of d taking half) and records 2^-c.
  const int d = tid >> 1;
  char* vdst = dst + P * kPlaneBytes;
  int cx = 0;
  if constexpr (P == 2) {
    float amax = 0.f;
#pragma unroll 8
    for (int t = 32 * (tid & 1); t < 32 * (tid & 1) + 32; ++t) amax = fmaxf(amax, fabsf(vt[t][d]));
    cx = scale_exponent(fmaxf(amax, __shfl_xor(amax, 1, 64)));
    if ((tid & 1) == 0) *reinterpret_cast<float*>(dst + kVScaleOffset + 4 * d) = ldexpf(1.0f, -cx);
  }
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    const int c = 4 * (tid & 1) + cc;
    V8 hi, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      split2v<E>(P == 2 ? ldexpf(vt[vt_pos_m<MODE>(c, j)][d], cx) : vt[vt_pos_m<MODE>(c, j)][d], hi, lo, j);
    *reinterpret_cast<V8*>(vdst + vt_off(d, c)) = hi;
    if constexpr (P == 2) *reinterpret_cast<V8*>(vdst + kPlaneBytes + vt_off(d, c)) = lo;
  }
}

// Partial layout per (kv head, row block, split): O in 16-byte chunks
// (128 columns x kD floats), chunk (8 cb + b) * 64 + l holding O^T[16 b + 4
// (l / 16) .. + 3][16 cb + l % 16] (lane l's four values of d block b for
// column block cb: the writer's 64 lanes store 1 KiB contiguous), then
// (max, sum)[128 columns].
constexpr size_t kPartStride = (size_t)128 * kD + 2 * 128;

// Units of a launch: (split, row block, kv head) of a unit index, by
// blockIdx (each XCD a contiguous run, kv-head-major).
struct Unit {
  int split, rb, kvh;
  bool live;
};
__device__ __forceinline__ Unit unit_of(int n_units, int n_rb, int kv_splits) {
  // Workgroups are dispatched round-robin over the 8 XCDs (block b runs on
  // XCD b % 8). Units (kv head, row block, split) are numbered kv-head-major
  // and each XCD takes a contiguous run of them, so the workgroups sharing
  // an XCD's L2 stream the same kv head's tiles at about the same time.
  // With a KV split the row blocks go last-first within a kv head, so each
  // XCD dispatches its longest ranges first (config 4 93.7 -> 91.5 us);
  // without one they go first-first: the short units then read the first
  // tiles into the XCD's L2 ahead of the long ones (last-first cost config
  // 3 +0.3 us).
  Unit u;
  const int per_xcd = (n_units + 7) / 8;
  const int unit = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  u.live = (int)(blockIdx.x / 8) < per_xcd && unit < n_units;
  u.split = unit % kv_splits;
  u.rb = (unit / kv_splits) % n_rb;
  if (kv_splits > 1) u.rb = n_rb - 1 - u.rb;
  u.kvh = unit / (kv_splits * n_rb);
  return u;
}

// This lane's 32 elements of one query vector, d = 8 kk + 32 s + e, from qp
// (already offset by 8 kk), and with qn_w the q prologue's operands: the
// loads only (issue), so the caller can queue other loads behind them before
// anything waits; then (finish) the q prologue, as the row prologue would:
// RMSNorm with an f64 sum of squares over the column's four lanes (lanes 16
// and 32 apart), then `x * inv * w` and the rotation of the pairs (i, i +
// 64) - both in this lane, s and s + 2 - in the reference's separately
// rounded f32 operations, with the row's (cos, sin) from tab_row (64 cos,
// then 64 sin).
struct Q16Loads {
  float x[4][8];
  float w0[2][8], w1[2][8], cs[2][8], sn[2][8];
  __device__ __forceinline__ void issue(const float* qp, int kk, const float* __restrict__ qn_w,
                                        const float* __restrict__ tab_row) {
    // Rows, weights and table 16-byte aligned (the common case): 16-byte loads.
    const bool vec = aligned16(qp, qn_w, tab_row);
#pragma unroll
    for (int s = 0; s < 4; ++s) ld8(qp + 32 * s, vec, x[s]);
    if (!qn_w) return;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int i = 8 * kk + 32 * s;
      ld8(qn_w + i, vec, w0[s]);
      ld8(qn_w + i + 64, vec, w1[s]);
      ld8(tab_row + i, vec, cs[s]);
      ld8(tab_row + 64 + i, vec, sn[s]);
    }
  }
  // The operands from LDS instead: the weights at w (128 floats) and the
  // row's (cos, sin) at t.
  __device__ __forceinline__ void operands_from(const float* w, const float* t, int kk) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int i = 8 * kk + 32 * s;
      ld8(w + i, true, w0[s]);
      ld8(w + i + 64, true, w1[s]);
      ld8(t + i, true, cs[s]);
      ld8(t + 64 + i, true, sn[s]);
    }
  }
  __device__ __forceinline__ void finish(bool norm, float qn_eps) {
#pragma clang fp contract(off)
    if (!norm) return;
    double ss = 0.0;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (double)x[s][e] * (double)x[s][e];
    ss = swap_sum_f64<32>(swap_sum_f64<16>(ss));
    const float inv = (float)(1.0 / sqrt(ss / (double)kD + (double)qn_eps));
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a0 = x[s][e] * inv * w0[s][e], a1 = x[s + 2][e] * inv * w1[s][e];
        x[s][e] = a0 * cs[s][e] - a1 * sn[s][e];
        x[s + 2][e] = a0 * sn[s][e] + a1 * cs[s][e];
      }
  }
};

// NaN-propagating max of three (v_maximum3_f32: unlike fmaxf it needs no
// operand canonicalisation).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Sum of the 8 P values of a B operand in fp32 (v_dot2 with (1, 1)): the
// softmax denominator of exactly the rounded P the PV products use.
__device__ __forceinline__ float sum8(f16x8 v, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 0, 1), h2{1, 1}, acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 2, 3), h2{1, 1}, acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 4, 5), h2{1, 1}, acc, false);
  return __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 6, 7), h2{1, 1}, acc, false);
}
__device__ __forceinline__ float sum8(bf16x8 v, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 one = {(__bf16)1.0f, (__bf16)1.0f};
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), one, acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), one, acc, false);
}

// The sum of P values i and i + 1 of a B operand added to acc (one v_dot2).
__device__ __forceinline__ float sum2(f16x8 v, int i, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(h2{v[i], v[i + 1]}, h2{1, 1}, acc, false);
}
__device__ __forceinline__ float sum2(bf16x8 v, int i, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(b2{v[i], v[i + 1]}, one, acc, false);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// p - h[i] for the f16 pair h, exactly (p - h is representable when h is p
// rounded to f16): one v_fma_mix_f32 reading the f16 half in place, where
// converting h to f32 and subtracting takes two instructions.
template <int I>
__device__ __forceinline__ float residual_f16(f16x2 h, float p) {
  float r;
  if constexpr (I == 0)
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(p));
  else
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(p));
  return r;
}

// prefill_kernel (the split mode): one group of W = 4 waves; column m of the
// workgroup's M = 16 W MT is head m / qr, row m % qr of the block (qr = M /
// group), wave w owning columns [16 MT w, 16 MT (w + 1)). A tile is 68 KiB
// (K hi, K lo, V^T hi, V^T lo planes, then the exponents) and the ring holds
// two. The loop is software-pipelined inside each wave, as the F16 / BF16
// kernel's: iteration j exponentiates and splits tile j's P between the
// MFMAs of tile j + 1's scores (phase A), then scales tile j + 1's scores and
// takes their maximum between tile j's PV MFMAs (phase B), each chunk fenced
// so the compiler keeps that issue order; the shadow of the MFMAs holds the
// softmax work, which otherwise ran between the MFMA phases on the SIMD's
// single wave. Tile j + 2's K half and tile j + 1's V half are copied in
// early in phase A, into the halves of the ring the previous iteration
// finished with.
template <int MODE, int G, int W, int MT, int NS>
__global__ __launch_bounds__(G * W * 64) void prefill_kernel(const float* __restrict__ q,
                                                             const char* __restrict__ stage, int n_stage_tiles,
                                                             int q_stride, int rows, int start, int group, int n_rb,
                                                             int n_units, int kv_splits, float qscale,
                                                             const float* __restrict__ qn_w, float qn_eps,
                                                             const float* __restrict__ qn_tab,
                                                             float* __restrict__ part, float* __restrict__ out) {
  typedef typename Op<MODE>::E E;
  typedef typename Op<MODE>::V8 V8;
  typedef typename Op<MODE>::V4 V4;
  constexpr bool kSplit = Op<MODE>::kSplit;
  static_assert(kSplit && G == 1 && NS == 2 && (W == 4 || W == 8), "the split mode: one group of 4 or 8 waves, two stages");
  // (8 waves of 16 columns measured equal to 4 waves of 32 at config 4.)
  constexpr int NPL = 32 / W;  // plane pieces per wave per half tile
  constexpr int M = 16 * W * MT;       // query vectors per workgroup
  constexpr int TB = kTileBytes<MODE>;  // bytes per staged tile
  static_assert(TB == 68 * 1024 && kVScaleOffset == kScaleOffset + 1024, "68 pieces of 1 KiB");
  // Scores are kept relative to a running maximum that only moves when a
  // tile's maximum exceeds it by more than this (log2 units): P values stay
  // below 2^8 and most tiles skip rescaling the accumulators.
  constexpr float kRescale = 8.0f;

  __shared__ __attribute__((aligned(1024))) char lds[NS][TB];

  const int tid = threadIdx.x, lane = tid & 63;
  const Unit un = unit_of(n_units, n_rb, kv_splits);
  if (!un.live) return;
  const int split = un.split, rb = un.rb, kvh = un.kvh;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lm = lane & 15, kk = lane >> 4;
  const int qr = M / group;  // rows per workgroup
  const int r0 = rb * qr;
  const int rows_here = min(qr, rows - r0);
  const int wg_limit = start + r0 + rows_here;  // positions the block's last row sees
  const int all_see = start + r0 + 1;           // positions every row of the block sees
  const int n_tiles = (wg_limit + kBT - 1) / kBT;
  const int tt_lo = (int)((long)n_tiles * split / kv_splits);
  const int n = (int)((long)n_tiles * (split + 1) / kv_splits) - tt_lo;

  // Half h of tile t (0: the K planes, pieces 0-31, and the K factors,
  // piece 64; 1: the V planes, 32-63, and the V factors, 65) into stage s,
  // in NPL + 1 parts per wave (NPL = 32 / W): part i < NPL is piece 32 h + w
  // + W i, part NPL piece 64 + h + 2 (w & 1) (even waves all copy the
  // factors, odd waves an unused piece: no branch). Lane l's 16 bytes land at piece + 16 l. A
  // half's global and LDS bases are wave-uniform, set once per half and
  // hidden from the compiler (so it computes each part's address where the
  // part is issued, instead of holding every part's address in scalar
  // registers across the loop). Tile indices are clamped to the range's last
  // tile, so the copies stay unconditional (past the range they refill a
  // half that nothing reads again).
  const char* const srcw = stage + ((size_t)kvh * n_stage_tiles + tt_lo) * TB;
  const uint32_t voff = 16u * (uint32_t)lane;
  struct HalfBase {
    const char* g;
    uint32_t l;
  };
  auto half_base = [&](int t, int s, int h) {
    HalfBase b{srcw + (size_t)min(t, n - 1) * TB + 1024 * (32 * h + wv),
               (uint32_t)lds_offset(&lds[s][1024 * (32 * h + wv)])};
    asm volatile("" : "+s"(b.g), "+s"(b.l));
    return b;
  };
  auto copy_part = [&](const HalfBase& b, int h, int i) {
    const int off = i < NPL ? 1024 * W * i : 1024 * (64 + h + 2 * (wv & 1) - 32 * h - wv);
    lds_dma16s(b.g + off, voff, b.l + off);
  };
  // This lane's query vector in column block mt: column m = 16*(wv*MT + mt) + lm.
  int my_row[MT], my_head[MT], my_limit[MT];
  bool col_ok[MT];
  Q16Loads qld[MT];
  // With the q prologue, its operands (the block's (cos, sin) rows, then the
  // norm weights) are copied once per workgroup into LDS (stage 1's V half,
  // unused until the loop) by a few coalesced copies, instead of every lane
  // loading its own: those scattered per-lane loads took ~4 us to issue at
  // 32 columns per wave. Unaligned operands or blocks of more than 48 rows
  // load per lane.
  // Row r of the table sits at float 260 r (1040 bytes: each row takes a
  // copy of its own, and the 16-byte skew puts the 16 rows one read
  // gathers on distinct banks), the weights after the rows.
  const bool pro_lds = qn_w != nullptr && aligned16(qn_w, qn_tab) && qr <= 30;
  float* const pro = reinterpret_cast<float*>(&lds[1][2 * kPlaneBytes]);
  constexpr int kProRow = 260;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * (wv * MT + mt) + lm;
    my_head[mt] = m / qr;
    my_row[mt] = r0 + m % qr;
    col_ok[mt] = my_row[mt] < rows && my_head[mt] < group;
    my_limit[mt] = col_ok[mt] ? start + my_row[mt] + 1 : 0;
    const int q_row = col_ok[mt] ? my_row[mt] : 0;
    qld[mt].issue(q + (size_t)q_row * q_stride + (size_t)(kvh * group + (col_ok[mt] ? my_head[mt] : 0)) * kD + 8 * kk,
                  kk, pro_lds ? nullptr : qn_w, pro_lds || !qn_tab ? nullptr : qn_tab + (size_t)q_row * kD);
  }
  if (pro_lds) {
    // Copy i: table row i of the block (512 bytes, twice: the second half
    // lands in the row's padding; rows past the chunk read its last), the
    // weights after the rows (wave 0).
    for (int i = wv; i < qr; i += W)
      lds_dma16(qn_tab + (size_t)min(r0 + i, rows - 1) * kD + 4 * (lane & 31), lds_offset(pro + kProRow * i));
    if (wv == 0) lds_dma16(qn_w + 4 * (lane & 31), lds_offset(pro + kProRow * qr));
  }
  // Tile 0's K half, queued behind the query loads (which return first, so
  // the q prologue runs while it lands). Tile 0's V half and tile 1's K
  // half are issued among tile 0's score MFMAs: issued here, their copies
  // held the wave ~2.5 us (the memory pipeline is full at the start, and a
  // wave issues in order) before it could start the q prologue.
  if (n > 0) {
    const HalfBase k0 = half_base(0, 0, 0);
#pragma unroll
    for (int i = 0; i <= NPL; ++i) copy_part(k0, 0, i);
  }
  if (pro_lds) {
    // The operand copies are done once only the tile copies may remain.
    if (n > 0)
      wait_vmcnt<NPL + 1>();
    else
      wait_vmcnt<0>();
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      qld[mt].operands_from(pro + kProRow * qr, pro + kProRow * (my_row[mt] - r0), kk);
  }

  V8 qh[MT][4], ql[MT][4];
  // log2(e) * scale * 2^-qe: undoes the vector's exponent qe and scales its
  // fp32 scores.
  float qf[MT];
  f32x4 o[MT][8];
  float m_run[MT], l_run[MT];
  // -m_run, or 0 while a column has seen no unmasked position: added to the
  // scores after scaling, so they are relative to the running max.
  float negm[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    // The scores are scaled by log2(e) * scale in fp32 (rounding the scaled
    // q would cost low bits of the lo half).
    const float qs = col_ok[mt] ? 1.f : 0.f;
    qld[mt].finish(qn_w != nullptr, qn_eps);
    const float(&x)[4][8] = qld[mt].x;
    // The vector scaled by its exponent (from its max over the column's four
    // lanes), undone on the fp32 scores; capped at 100 so qscale * 2^-qe
    // stays a normal float (a vector below 2^-86 throughout keeps its
    // largest elements in f16's range and contributes scores below 2^-60).
    float amax = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[s][e] * qs));
    const int qe = scale_exponent(swap_max<32>(swap_max<16>(amax)), 100);
    qf[mt] = ldexpf(qscale, -qe);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) split2v<E>(ldexpf(x[s][e] * qs, qe), qh[mt][s], ql[mt][s], e);
      // Held in AGPRs: the QK MFMAs read them from there, which leaves the
      // VGPRs to the loop's working set.
      asm("" : "+a"(qh[mt][s]));
      asm("" : "+a"(ql[mt][s]));
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) o[mt][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[mt] = kNegSentinel;
    l_run[mt] = 0.f;
    negm[mt] = 0.f;
  }

  if (n > 0) {
    typedef __attribute__((address_space(3))) const char* LdsPtr;
    // Scores of a tile: s[mt][pb][e] = S^T[16 pb + 4 kk + e][column block mt];
    // element i = 4 (MT pb + mt) + e in the orders below.
    typedef f32x4 Scores[MT][4];
    // Per-lane LDS bases per stage (stage 1 lies past the reads' 16-bit
    // immediate offsets, so each stage gets its own): K row lm at d chunk
    // 4 ks + kk; V^T row lm at chunk 4 s2 + kk; this lane's four K factors
    // (positions 4 kk .. + 3 of a 16-position block) and V^T factors.
    // Every read below is one of these plus an immediate.
    LdsPtr kb[2][4], vb[2][2], kfb[2], vfb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const LdsPtr st = (LdsPtr)&lds[s][0];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        kb[s][ks] = st + k_off(lm, 4 * ks + kk);
        asm("" : "+v"(kb[s][ks]));
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        vb[s][s2] = st + 2 * kPlaneBytes + vt_off(lm, 4 * s2 + kk);
        asm("" : "+v"(vb[s][s2]));
      }
      kfb[s] = st + kScaleOffset + 16 * kk;
      vfb[s] = st + kVScaleOffset + 16 * kk;
      asm("" : "+v"(kfb[s]));
      asm("" : "+v"(vfb[s]));
    }
    // K operands of QK chunk c = (pb, ks), pb-major: rows 16 pb + lm, d
    // chunk 4 ks + kk (the swizzle k_off depends on the row only through lm),
    // both planes.
    auto kread = [&](int s, int c, V8& a, V8& al) {
      const LdsPtr p = kb[s][c & 3] + 4096 * (c >> 2);
      a = *reinterpret_cast<const __attribute__((address_space(3))) V8*>(p);
      al = *reinterpret_cast<const __attribute__((address_space(3))) V8*>(p + kPlaneBytes);
    };
    // Chunk c's three split products (hi·hi, lo·hi, hi·lo) for every column
    // block, into fresh accumulators at ks = 0.
    auto qk_chunk = [&](int c, const V8& a, const V8& al, Scores& s) {
      const int pb = c >> 2, ks = c & 3;
      if (ks == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) s[mt][pb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) s[mt][pb] = Op<MODE>::mfma(a, qh[mt][ks], s[mt][pb]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) s[mt][pb] = Op<MODE>::mfma(al, qh[mt][ks], s[mt][pb]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) s[mt][pb] = Op<MODE>::mfma(a, ql[mt][ks], s[mt][pb]);
    };
    // A tile's 16 QK chunks from stage st with a ring of three K operand
    // reads; between(c) runs in chunk c, each chunk fenced.
    auto qk_tile = [&](int st, Scores& s, auto between) {
      V8 ka[3], kal[3];
      kread(st, 0, ka[0], kal[0]);
      kread(st, 1, ka[1], kal[1]);
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        if (c + 2 < 16) kread(st, c + 2, ka[(c + 2) % 3], kal[(c + 2) % 3]);
        qk_chunk(c, ka[c % 3], kal[c % 3], s);
        between(c);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // Causal mask of tile jj's scores, only where some row of the block stops
    // inside the tile.
    auto mask = [&](int jj, Scores& s) {
      const int t0 = (tt_lo + jj) * kBT;
      if (t0 + kBT > all_see) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int pb = 0; pb < 4; ++pb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (t0 + 16 * pb + 4 * kk + e >= my_limit[mt]) s[mt][pb][e] = -INFINITY;
      }
    };
    // The K factors 2^-e_t of positions 16 pb + 4 kk + e.
    auto read_kf = [&](int s, int pb) {
      return *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(kfb[s] + 64 * pb);
    };
    // Elements i and i + 1 (one column block) of s: the K row and q
    // exponents undone (exact powers of two), the fp32 scale and -max
    // applied, both into that column's running maximum of the tile.
    auto scale_pair = [&](Scores& s, const f32x4& kf, int i, float (&mx)[MT]) {
      const int pb = i / (4 * MT), mt = (i / 4) % MT, e = i % 4;
      s[mt][pb][e] = __builtin_fmaf(s[mt][pb][e] * kf[e], qf[mt], negm[mt]);
      s[mt][pb][e + 1] = __builtin_fmaf(s[mt][pb][e + 1] * kf[e + 1], qf[mt], negm[mt]);
      mx[mt] = max3f(mx[mt], s[mt][pb][e], s[mt][pb][e + 1]);
    };
    // Online softmax step of a tile whose scores are scaled and whose lane
    // maxima are mx: the column maxima across the column's four lanes (16
    // and 32 apart, permlane swaps); a column still at the sentinel takes the
    // tile's maximum outright (its O and sum are zero), others move up by d
    // >= 0 and rescale, only when some column of the wave grows by more than
    // kRescale.
    auto adjust = [&](float (&mx)[MT], Scores& s) {
      bool grow = false;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float x = mx[mt];
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __builtin_elementwise_maximum(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        mx[mt] = __builtin_elementwise_maximum(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
        grow = grow || mx[mt] > kRescale || m_run[mt] == kNegSentinel;
      }
      if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const bool fresh = m_run[mt] == kNegSentinel;
          const float d = fresh ? fmaxf(mx[mt], kNegSentinel) : fmaxf(mx[mt], 0.f);
          if (!fresh) {
            const float alpha = __builtin_amdgcn_exp2f(-d);
            l_run[mt] *= alpha;
#pragma unroll
            for (int b = 0; b < 8; ++b) o[mt][b] *= alpha;
            m_run[mt] += d;
          } else {
            m_run[mt] = d;
          }
#pragma unroll
          for (int pb = 0; pb < 4; ++pb) s[mt][pb] -= d;
          negm[mt] = m_run[mt] == kNegSentinel ? 0.f : -m_run[mt];
        }
      }
    };
    // P^T operands of PV step s2: slots j < 4 are t = 32 s2 + 4 kk + j, slots
    // j >= 4 are t = 32 s2 + 16 + 4 kk + j - 4 (blocks 2 s2 and 2 s2 + 1),
    // as f16 hi + lo of P (< 2^8).
    typedef V8 POps[MT][2];
    // Each exponential and split is pinned where it is written by an empty
    // volatile asm (otherwise they are sunk past the mask's branch to the PV
    // MFMAs that use them).
    auto exp_el = [&](Scores& s, int i) {
      const int pb = i / (4 * MT), mt = (i / 4) % MT, e = i % 4;
      s[mt][pb][e] = __builtin_amdgcn_exp2f(s[mt][pb][e]);
      asm volatile("" : "+v"(s[mt][pb][e]));
    };
    // Group g = MT pb + mt of exponentials (done) into the P operands.
    auto split_grp = [&](const Scores& s, int g, POps& ph, POps& pl) {
      const int pb = g / MT, mt = g % MT;
      const f32x4 p = s[mt][pb];
      V4 hi = __builtin_convertvector(p, V4);
      const f16x2 h01 = {hi[0], hi[1]}, h23 = {hi[2], hi[3]};
      const f32x4 r = {residual_f16<0>(h01, p[0]), residual_f16<1>(h01, p[1]), residual_f16<0>(h23, p[2]),
                       residual_f16<1>(h23, p[3])};
      V4 lo = __builtin_convertvector(r, V4);
      asm volatile("" : "+v"(hi), "+v"(lo));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ph[mt][pb / 2][4 * (pb % 2) + e] = hi[e];
        pl[mt][pb / 2][4 * (pb % 2) + e] = lo[e];
      }
    };
    // Share b (of 8) of the column sums of P as the PV products use it (hi
    // + lo), into l_run: term k of column block mt is the pair k % 4 of
    // plane (k / 4) % 2 (hi, lo) of step k / 8, one v_dot2 each. It runs
    // among the PV MFMAs, whose half of the loop has VALU to spare.
    auto sum_share = [&](const POps& ph, const POps& pl, int b) {
#pragma unroll
      for (int u = 0; u < 2 * MT; ++u) {
        const int idx = 2 * MT * b + u, mt = idx / 16, k = idx % 16;
        const V8& v = ((k >> 2) & 1) ? pl[mt][k >> 3] : ph[mt][k >> 3];
        l_run[mt] = sum2(v, 2 * (k & 3), l_run[mt]);
      }
    };
    // O^T += V^T P^T from stage st in 8 fenced d blocks b: block b's 6 MT
    // MFMAs (two steps, the three split products, into a fresh accumulator;
    // the V operands of step h = 2 b + s2 read two steps ahead), block b +
    // 1's V factors, block b - 1's fold into O with its factors (this lane's
    // O^T rows are d = 16 b + 4 kk + e), and between(b).
    auto pv_tile = [&](int st, const POps& ph, const POps& pl, auto between) {
      V8 va[3], val[3];
      f32x4 cf[3];
      auto vread = [&](int h) {
        const LdsPtr p = vb[st][h & 1] + 2048 * (h >> 1);
        va[h % 3] = *reinterpret_cast<const __attribute__((address_space(3))) V8*>(p);
        val[h % 3] = *reinterpret_cast<const __attribute__((address_space(3))) V8*>(p + kPlaneBytes);
      };
      auto cread = [&](int b) {
        cf[b % 3] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(vfb[st] + 64 * b);
      };
      f32x4 pend[MT];
      auto fold = [&](int b) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) o[mt][b][e] = __builtin_fmaf(pend[mt][e], cf[b % 3][e], o[mt][b][e]);
      };
      vread(0);
      vread(1);
      cread(0);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        f32x4 acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int h = 2 * b + s2;
          if (h + 2 < 16) vread(h + 2);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[mt] = Op<MODE>::mfma(va[h % 3], ph[mt][s2], acc[mt]);
            acc[mt] = Op<MODE>::mfma(val[h % 3], ph[mt][s2], acc[mt]);
            acc[mt] = Op<MODE>::mfma(va[h % 3], pl[mt][s2], acc[mt]);
          }
        }
        if (b + 1 < 8) cread(b + 1);
        if (b > 0) fold(b - 1);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) pend[mt] = acc[mt];
        between(b);
        // Issue order inside the block: its LDS reads, two MFMAs, then two
        // VALU instructions after each further MFMA (left to itself the
        // scheduler put block b - 1's fold right behind the block's first
        // MFMA, waiting on block b - 1's last; this order measured ~10 %
        // faster for the half).
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // DS reads
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
#pragma unroll
        for (int i = 0; i < 6 * MT - 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      fold(7);
    };

    // Tile 0: scores, mask, scaling and maximum on their own, once its K
    // half has landed; its V half and tile 1's K half are copied in among
    // the score MFMAs (the first iteration waits for them).
    Scores sA, sB;
    wait_vmcnt<0>();
    __syncthreads();
    {
      const HalfBase v0 = half_base(0, 0, 1), k1 = half_base(1, 1, 0);
      qk_tile(0, sA, [&](int c) {
        if (c <= NPL) copy_part(v0, 1, c);
        if (c >= 7 && c <= 7 + NPL) copy_part(k1, 0, c - 7);
      });
      mask(0, sA);
      float mx[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) mx[mt] = -INFINITY;
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const f32x4 kf = read_kf(0, pb);
#pragma unroll
        for (int u = 0; u < 4 * MT; u += 2) scale_pair(sA, kf, 4 * MT * pb + u, mx);
      }
      adjust(mx, sA);
    }
    // One iteration jj of parity P (tile jj in stage P, tile jj + 1's K half
    // in stage 1 - P): scores sc of tile jj in (scaled, adjusted), scores sn
    // of tile jj + 1 out (scaled, adjusted).
    auto iter = [&](int jj, Scores& sc, Scores& sn, auto par_c) {
      constexpr int P = decltype(par_c)::value;
      wait_vmcnt<0>();  // tile jj's V half and tile jj + 1's K half
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      POps ph, pl;
      // Phase A: tile jj + 1's QK chunks; chunk c takes MT of tile jj's
      // exponentials and splits the groups whose exponentials an earlier
      // chunk finished. Tile jj + 2's K half (needed first, at the next
      // iteration's start) and then tile jj + 1's V half are copied in over
      // the first chunks, so every copy has most of the iteration to land
      // before the next iteration's wait.
      const HalfBase kh = half_base(jj + 2, P, 0), vh = half_base(jj + 1, 1 - P, 1);
      qk_tile(1 - P, sn, [&](int c) {
#pragma unroll
        for (int u = 0; u < MT; ++u) exp_el(sc, MT * c + u);
#pragma unroll
        for (int g = 0; g < 4 * MT; ++g)
          if ((4 * g + 3) / MT + 1 == c) split_grp(sc, g, ph, pl);
        if (c <= NPL) copy_part(kh, 0, c);
        if (c >= 1 && c <= NPL + 1) copy_part(vh, 1, c - 1);
      });
#pragma unroll
      for (int g = 0; g < 4 * MT; ++g)
        if ((4 * g + 3) / MT + 1 >= 16) split_grp(sc, g, ph, pl);
      mask(jj + 1, sn);
      // Phase B: tile jj's PV blocks; block b scales 2 MT of tile jj + 1's
      // scores into their maximum (K factors read a block ahead).
      float mx[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) mx[mt] = -INFINITY;
      f32x4 kf[4];
      kf[0] = read_kf(1 - P, 0);
      pv_tile(P, ph, pl, [&](int b) {
        sum_share(ph, pl, b);
        if ((b & 1) && b + 1 < 8) kf[(b + 1) / 2] = read_kf(1 - P, (b + 1) / 2);
#pragma unroll
        for (int u = 0; u < 2 * MT; u += 2) scale_pair(sn, kf[b / 2], 2 * MT * b + u, mx);
      });
      adjust(mx, sn);
    };
    // The last tile: its P and PV MFMAs only.
    auto last = [&](Scores& sc, auto par_c) {
      constexpr int P = decltype(par_c)::value;
      wait_vmcnt<0>();
      __syncthreads();
      POps ph, pl;
#pragma unroll
      for (int i = 0; i < 16 * MT; ++i) exp_el(sc, i);
#pragma unroll
      for (int g = 0; g < 4 * MT; ++g) split_grp(sc, g, ph, pl);
      pv_tile(P, ph, pl, [&](int b) { sum_share(ph, pl, b); });
    };
    int j = 0;
    for (; j + 2 < n; j += 2) {
      iter(j, sA, sB, std::integral_constant<int, 0>{});
      iter(j + 1, sB, sA, std::integral_constant<int, 1>{});
    }
    if (j + 1 < n) {
      iter(j, sA, sB, std::integral_constant<int, 0>{});
      last(sB, std::integral_constant<int, 1>{});
    } else {
      last(sA, std::integral_constant<int, 0>{});
    }
  }
  // Every copy has landed (the last tile's step issues none); retire them
  // before the workgroup ends.
  wait_vmcnt<0>();

  // Column sums: each lane holds a quarter of its column's positions.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    l_run[mt] += __shfl_xor(l_run[mt], 16, 64);
    l_run[mt] += __shfl_xor(l_run[mt], 32, 64);
  }

  if (kv_splits == 1) {
    // Non-temporal stores: nothing reads the output in this launch, and
    // lines already on their way out leave less for the end-of-kernel
    // write-back (config 3: 19.0 -> 18.6 us).
    const bool vec = aligned16(out) && q_stride % 4 == 0;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!col_ok[mt]) continue;
      const float inv = 1.0f / l_run[mt];
      float* op = out + (size_t)my_row[mt] * q_stride + (size_t)(kvh * group + my_head[mt]) * kD + 4 * kk;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const f32x4 y = o[mt][b] * inv;
        if (vec) {
          __builtin_nontemporal_store(y, reinterpret_cast<f32x4*>(op + 16 * b));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) __builtin_nontemporal_store(y[e], op + 16 * b + e);
        }
      }
    }
    return;
  }
  // Partial (O, max, sum) of this split; o[mt][b][e] is O^T[16b + 4kk + e][m].
  float* mine = part + (((size_t)kvh * n_rb + rb) * kv_splits + split) * kPartStride;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * (wv * MT + mt) + lm;
#pragma unroll
    for (int b = 0; b < 8; ++b) reinterpret_cast<f32x4*>(mine)[((wv * MT + mt) * 8 + b) * 64 + lane] = o[mt][b];
    if (kk == 0) {
      mine[128 * kD + 2 * m] = m_run[mt];
      mine[128 * kD + 2 * m + 1] = l_run[mt];
    }
  }
}

// ---- F16 / BF16: v_mfma_f32_32x32x16 tiles --------------------------------------------
//
// prefill32_kernel<MODE, W, G>: one workgroup of W waves per (kv head, block
// of V = 32 W / G query vectors, KV split), in G groups of W / G waves; wave
// wv of each group owns the 32 columns [32 wv, 32 wv + 32) (column m is head
// m / qr, row m % qr of the block, qr = V / group). Group gi computes the
// tiles G j + gi of the workgroup's range for its columns, and the groups'
// (O, max, sum) merge through LDS at the end, so one step of the ring feeds
// V columns from each of G tiles and the causal chain of the block's longest
// range is 1 / G as long. Each operand read feeds an MFMA of 32 columns
// (twice the columns per LDS byte of a 16x16 tile). The instantiation is
// W = 8, G = 2: 128-column units, the same throughput at 3.9k positions as 256-column
// units with twice the KV splits (47.1 vs 48.3 us), and a chain half as long
// where the chunk's own rows dominate (config 3: 14.4 vs 16.0 us). Per
// tile, per wave:
//   S^T[t][m] = sum_d K[t][d] Q[m][d]: A = K (32 positions x 16 d, one
//     16-byte chunk of a staged K row per lane), B = Q^T (this lane's column
//     lc = lane % 32 at d = 16 ks + 8 g + i, g = lane / 32), in registers;
//     2 position blocks x 8 d steps = 16 MFMAs into two 32x32 accumulators
//     started at -max (scores arrive relative to the running maximum);
//   lane (lc, g) then holds rows 32 pb + 8 (r / 4) + 4 g + r % 4 of column
//     lc in register r: the column's maximum is this lane's 32 values and its
//     partner's (one permlane32 swap), and registers 8 h .. 8 h + 7 of block
//     pb, rounded, are exactly the B operand P^T of PV step (pb, h) (the V^T
//     tile is staged with its positions in that order, vt_pos32);
//   O^T[d][m] += sum_t V^T[d][t] P^T[t][m]: 4 d blocks x 4 steps = 16 MFMAs.
// The loop is software-pipelined inside each wave: tile j's exponentials run
// between the MFMAs of tile j + 1's scores and tile j + 1's maximum between
// tile j's PV MFMAs, written out chunk by chunk in issue order. On gfx950 an
// MFMA 32x32x16 hides only about four full-rate VALU instructions (two
// exponentials) of the same SIMD; a phase of softmax work between phases of
// MFMAs costs its full length (measured: the two waves of a SIMD run their
// phases in step, so the other wave does not fill the gap). Tiles stream
// through a 4-stage ring by direct-to-LDS loads (inline assembly, so the
// compiler adds no wait for them before LDS reads), the next step's planes
// in flight during a step. The KV range is split across
// workgroups when the chunk has too few query
// blocks to fill the chip; the splits of a block run on one XCD (blockIdx
// agreeing mod 8: the dispatcher deals workgroups to the XCDs round robin),
// write their partial (O, max, sum) columns with plain stores and take a
// ticket, and the last to finish folds them in split order from that XCD's
// L2 (no second launch, no workgroup waits on another).
constexpr int kP32Stages = 4;
constexpr int kP32Waves = 8;   // per workgroup
constexpr int kP32Groups = 2;  // wave groups splitting a unit's tiles
static_assert(32 * kP32Waves / kP32Groups == kQPrepVectors, "unit columns");
constexpr int kP32TileBytes = 2 * kPlaneBytes;
constexpr int kP32Part = 130;  // floats per partial column: O[128], max, sum
constexpr int kPolicyL2 = 1;   // the sc0 bit: the load misses the CU's L1 and reads its XCD's L2

template <int MODE>
struct Op32;
template <>
struct Op32<kF16> {
  __device__ static f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Op32<kBF16> {
  __device__ static f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// The last split's fold of a unit's columns over its S splits, d blocks DB0
// and DB0 + 1 (32 d each): split sp's partial column (O chunks 8 db + 2 jj +
// g of this lane from o_off(sp, chunk), max and sum from ml_off(sp); split
// `own`, the folding one, from its registers oo, m_own, l_own, which hold
// exactly what it stored), weighted by 2^(max_sp - M) over M = the splits'
// maximum and summed in split order; emit(db, block, 1 / L) for each block.
// S is fixed at compile time so the loads are issued without data-dependent
// branches; up to 4 splits every load is issued before the first is used.
template <int S, int DB0, typename OffFn, typename MlFn, typename Emit>
__device__ __forceinline__ void fold32(const __amdgpu_buffer_rsrc_t& rs, OffFn o_off, MlFn ml_off, int g,
                                       Emit emit, int own, const f32x16 (&oo)[4], float m_own, float l_own) {
  constexpr int NB = S <= 4 ? 2 : 1;  // blocks in flight
  f32x4 buf[NB][S][4];
  auto load_block = [&](auto bkc, f32x4 (&b)[S][4]) {
    constexpr int db = DB0 + decltype(bkc)::value;
#pragma unroll
    for (int sp = 0; sp < S; ++sp)
      if (sp != own) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          b[sp][jj] = __builtin_amdgcn_raw_buffer_load_b128(rs, o_off(sp, 8 * db + 2 * jj + g), 0, kPolicyL2);
      } else {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          b[sp][jj] = f32x4{oo[db][4 * jj], oo[db][4 * jj + 1], oo[db][4 * jj + 2], oo[db][4 * jj + 3]};
      }
  };
  float ms[S], ls[S];
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
    if (sp != own) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, ml_off(sp), 0, kPolicyL2);
      ms[sp] = __builtin_bit_cast(float, (uint32_t)v[0]);
      ls[sp] = __builtin_bit_cast(float, (uint32_t)v[1]);
    } else {
      ms[sp] = m_own;
      ls[sp] = l_own;
    }
  }
  load_block(std::integral_constant<int, 0>{}, buf[0]);
  if constexpr (NB == 2) load_block(std::integral_constant<int, 1>{}, buf[NB - 1]);
  float M = ms[0];
#pragma unroll
  for (int sp = 1; sp < S; ++sp) M = fmaxf(M, ms[sp]);
  float a[S], L = 0.f;
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
    a[sp] = __builtin_amdgcn_exp2f(ms[sp] - M);
    L += ls[sp] * a[sp];
  }
  const float inv = 1.0f / L;
  auto fold_block = [&](const f32x4 (&cur)[S][4]) {
    f32x16 acc{};
#pragma unroll
    for (int sp = 0; sp < S; ++sp)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * jj + e] += cur[sp][jj][e] * a[sp];
    return acc;
  };
  emit(DB0, fold_block(buf[0]), inv);
  if constexpr (NB == 1) load_block(std::integral_constant<int, 1>{}, buf[0]);
  emit(DB0 + 1, fold_block(buf[NB - 1]), inv);
}

template <int MODE, int W, int G>
__global__ __launch_bounds__(64 * W) void prefill32_kernel(const float* __restrict__ q, const char* __restrict__ stage,
                                                        int n_stage_tiles, int q_stride, int rows, int start,
                                                        int group, int n_rb, int n_units, int per_xcd, int kv_splits,
                                                        float qscale, const float* __restrict__ qn_w, float qn_eps,
                                                        const float* __restrict__ qn_tab,
                                                        const char* __restrict__ qprep, float* __restrict__ part,
                                                        uint32_t part_bytes, unsigned* __restrict__ tickets,
                                                        float* __restrict__ out) {
  typedef typename Op<MODE>::E E;
  typedef typename Op<MODE>::V8 V8;
  constexpr int TB = kP32TileBytes, NS = kP32Stages;
  constexpr int VG = W / G;        // waves per group
  constexpr int V = 32 * VG;       // columns per unit
  // Scores may exceed the running maximum by 2^kRescale (log2 units) before
  // it moves: P stays below 2^8 and most tiles skip rescaling O.
  constexpr float kRescale = 8.0f;
  __shared__ __attribute__((aligned(1024))) char lds[NS][TB];
  __shared__ unsigned sm_ticket;
  __shared__ float sm_ml[4 * VG * 64];

  // Unit (kv head, row block) and split: the splits of a unit share blockIdx
  // mod 8 (one XCD); each XCD takes a contiguous run of units, kv-head-major,
  // so its L2 holds about one kv head's tiles.
  const int slot = (int)(blockIdx.x & 7), rest = (int)(blockIdx.x >> 3);
  const int split = rest % kv_splits, ui = rest / kv_splits;
  const int ud = slot * per_xcd + ui;  // dispatch order
  if (ui >= per_xcd || ud >= n_units) return;
  // With a KV split the row blocks go last-first within a kv head (each
  // XCD dispatches its longest ranges first; without a split the short
  // units warm the XCD's L2 with the first tiles instead, as in unit_of);
  // u is the unit's index in (kv head, row block) order, which the prepared
  // queries, the partials and the tickets use.
  const int kvh = ud / n_rb, rb = kv_splits > 1 ? n_rb - 1 - ud % n_rb : ud % n_rb;
  const int u = kvh * n_rb + rb;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = w / VG, wv = w % VG;  // group, wave within it
  const int g = lane >> 5, lc = lane & 31;
  const int qr = V / group;
  const int r0 = rb * qr, rows_here = min(qr, rows - r0);
  const int wg_limit = start + r0 + rows_here;  // positions the block's last row sees
  const int all_see = start + r0 + 1;           // positions every row of the block sees
  const int n_tiles = (wg_limit + kBT - 1) / kBT;
  const int tt_lo = (int)((long)n_tiles * split / kv_splits);
  const int n = (int)((long)n_tiles * (split + 1) / kv_splits) - tt_lo;
  const int m = 32 * wv + lc;  // this lane's column
  const int head = m / qr, row = r0 + m % qr;
  const bool col_ok = m % qr < rows_here;
  const int my_limit = start + row + 1;

  // The column's query vector: prepared by the chunk's row prologue (eight
  // 16-byte loads), or loaded and put through the q prologue here (loads
  // first, so they return ahead of the tiles'); then the first three tiles.
  Q32Loads ql;
  V8 qv[8];
  const int q_row = col_ok ? row : r0;
  if (qprep) {
    const V8* qp = reinterpret_cast<const V8*>(qprep) + ((size_t)u * VG + wv) * 8 * 64 + lane;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qv[ks] = qp[64 * ks];
  } else {
    ql.issue(q + (size_t)q_row * q_stride + (size_t)(kvh * group + head) * kD, g, qn_w,
             qn_tab ? qn_tab + (size_t)q_row * kD : nullptr);
  }
  // Tile t of the range lands in stage 2 (t % 2) + (t / 2) % 2 as 32
  // pieces of 1 KiB (wave w copies pieces w, w + W, w + 2W, w + 3W: two in
  // the K plane, two in the V plane), so each group's two stages are
  // adjacent and every operand read below is a per-lane base plus an
  // immediate offset. The tile's address is wave-uniform (scalar
  // registers), the lane's 16 bytes an offset. A tile past the range copies
  // the range's last tile into its stage (free at that point either way):
  // the copies stay unconditional, so the loop body has no branch between
  // its MFMAs. (The units of an XCD walk their tiles in the same order:
  // their requests for a tile meet in that XCD's L2. Rotated starting
  // points measured 1.5 us slower at config 4.)
  const char* const srcw = stage + ((size_t)kvh * n_stage_tiles + tt_lo) * TB + 1024 * w;
  const uint32_t voff = 16u * (uint32_t)lane;
  auto stage_of = [](int t) { return 2 * (t & 1) + ((t >> 1) & 1); };
  // A wave's pieces of a tile: NK in the K plane (i < NK), NK in the V plane.
  constexpr int NK = 16 / W;
  auto copy_piece = [&](int t, int i) {
    lds_dma16s(srcw + (size_t)min(t, n - 1) * TB + 1024 * W * i, voff,
               lds_offset(&lds[stage_of(t)][1024 * (w + W * i)]));
  };
  // The K planes of tiles 0 and 1 (the first scores need only them); the V
  // planes of tiles 0 and 1 and the K planes of tiles 2 and 3 are issued
  // among the first score MFMAs (issued here, their copies held each wave
  // in the prologue while the memory pipeline was full). A split with no
  // tiles (more splits than the unit has tiles) copies nothing.
  if (n > 0) {
#pragma unroll
    for (int t = 0; t < G; ++t)
#pragma unroll
      for (int i = 0; i < NK; ++i) copy_piece(t, i);
  }
  if (qprep) {
    if (!col_ok) {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qv[ks] = V8{};
    }
  } else {
    ql.finish(qn_w != nullptr, qn_eps);
    const float qs = col_ok ? qscale : 0.f;  // log2(e) * scale, before rounding to the MFMA type
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[ks][e] = (E)(ql.x[ks][e] * qs);
  }

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16{};
  float m_run = kNegSentinel, l_run = 0.f;
  float negm = 0.f;  // -m_run, or 0 while the column has seen no position
  const int steps = (n + G - 1) / G;
  {
    static_assert((W == 8 || W == 4) && G == 2 && NS == 4, "two tiles per step; a wave's K pieces w + W i, i < NK, then its V pieces");
    // Software-pipelined: iteration j exponentiates tile j's scores while the
    // MFMAs of tile j + 1's scores run, then takes tile j + 1's maximum while
    // tile j's PV MFMAs run, each chunk written out in issue order so a
    // wave's softmax work fills the shadow of its own MFMAs. Iteration j
    // reads the V planes of step j and the K planes of step j + 1 and copies
    // in the V planes of step j + 1 and the K planes of step j + 2 (into the
    // halves the previous iteration finished with). Two iterations per trip
    // of the loop, so the two score arrays alternate roles in place and each
    // stage's parity is known at compile time. A group whose tile lies past
    // the range (group 1 when n is odd) computes on the copy of the range's
    // last tile in its stage, fully masked: P = 0, nothing added.
    if (n > 0) {
      const char* kp[8];
      const char* vp[4];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) kp[ks] = &lds[2 * gi][0] + 256 * lc + 16 * ((2 * ks + g) ^ (lc & 15));
#pragma unroll
      for (int c = 0; c < 4; ++c) vp[c] = &lds[2 * gi][kPlaneBytes] + 128 * lc + 16 * ((2 * c + g) ^ ((lc >> 1) & 7));
      // Operand k of a tile in the group's stage of parity par: K rows
      // 32 (k / 8) + lc at d step k % 8; V^T rows 32 (k / 4) + lc at step k % 4.
      auto kread = [&](int par, int k) {
        return *reinterpret_cast<const V8*>(kp[k & 7] + TB * par + 8192 * (k >> 3));
      };
      auto vread = [&](int par, int k) {
        return *reinterpret_cast<const V8*>(vp[k & 3] + TB * par + 4096 * (k >> 2));
      };
      // Copy c (of 4 NK) of iteration jj: c < 2 NK the V pieces of step jj +
      // 1, else the K pieces of step jj + 2.
      auto copy = [&](int jj, int c) {
        const int t = c < 2 * NK ? G * (jj + 1) + c / NK : G * (jj + 2) + (c - 2 * NK) / NK;
        copy_piece(t, c < 2 * NK ? NK + c % NK : c % NK);
      };
      auto mask = [&](int jj, f32x16 (&s)[2]) {
        const int tl = G * jj + gi;
        const int t0 = tl < n ? (tt_lo + tl) * kBT : (1 << 29);
        if (t0 + kBT > all_see) {
#pragma unroll
          for (int pb = 0; pb < 2; ++pb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (t0 + 32 * pb + 8 * (r >> 2) + 4 * g + (r & 3) >= my_limit) s[pb][r] = -INFINITY;
        }
      };
      auto lane_max = [&](float mx) {
        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        return __builtin_elementwise_maximum(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
      };
      auto adjust = [&](float mx, f32x16 (&s)[2]) {
        if (__builtin_amdgcn_ballot_w64(mx > kRescale || m_run == kNegSentinel)) {
          const bool fresh = m_run == kNegSentinel;
          const float d = fresh ? fmaxf(mx, kNegSentinel) : fmaxf(mx, 0.f);
          if (!fresh) {
            const float alpha = __builtin_amdgcn_exp2f(-d);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
            m_run += d;
          } else {
            m_run = d;
          }
          s[0] -= d;
          s[1] -= d;
          negm = m_run == kNegSentinel ? 0.f : -m_run;
        }
      };
      // One full iteration jj of parity P: scores sc of tile jj in, scores
      // sn of tile jj + 1 out.
      auto iter = [&](int jj, f32x16 (&sc)[2], f32x16 (&sn)[2], auto par_c) {
        constexpr int P = decltype(par_c)::value;
        wait_vmcnt<0>();  // step jj's V planes and step jj + 1's K planes
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        V8 ph[2][2];
        // Phase A: MFMA k of tile jj + 1's scores (started at -max), the K
        // operand read for MFMA k + 4, and P pair k of tile jj (two
        // exponentials, one conversion), each chunk fenced.
        {
          V8 ka[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) ka[k] = kread(1 - P, k);
#pragma unroll
          for (int r = 0; r < 16; ++r) sn[0][r] = negm, sn[1][r] = negm;
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            sn[k >> 3] = Op32<MODE>::mfma(ka[k & 3], qv[k & 7], sn[k >> 3]);
            if (k + 4 < 16) ka[k & 3] = kread(1 - P, k + 4);
            const int qb = k >> 3, h = (k >> 2) & 1, i = 2 * (k & 3);
            ph[qb][h][i] = (E)__builtin_amdgcn_exp2f(sc[qb][8 * h + i]);
            ph[qb][h][i + 1] = (E)__builtin_amdgcn_exp2f(sc[qb][8 * h + i + 1]);
            // An empty asm consuming the pair keeps it here: otherwise it is
            // sunk past the mask's branch to the PV MFMAs.
            asm("" : "+v"(ph[qb][h]));
            // The K pieces first (needed first), 4 NK copies over the 16 chunks;
            // with 4 waves (one per SIMD) the V pieces go to the PV half,
            // which has room for them (config 3: 10.46 -> 10.28 us).
            if constexpr (NK == 2) {
              if (k & 1) copy(jj, (4 + (k >> 1)) & 7);
            } else {
              if (k < 8) copy(jj, 8 + k);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        mask(jj + 1, sn);
        // Phase B: PV MFMA k of tile jj, the V operand read for MFMA k + 4,
        // two of tile jj + 1's 32 scores into its running maximum, and pair k
        // of tile jj's P into the sum (in the order the pairs were made).
        float mx = -INFINITY;
        {
          V8 va[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) va[k] = vread(P, k);
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const int c = k & 3;
            o[k >> 2] = Op32<MODE>::mfma(va[c], ph[c >> 1][c & 1], o[k >> 2]);
            if (k + 4 < 16) va[c] = vread(P, k + 4);
            mx = max3f(mx, sn[k >> 3][2 * (k & 7)], sn[k >> 3][2 * (k & 7) + 1]);
            l_run = sum2(ph[k >> 3][(k >> 2) & 1], 2 * (k & 3), l_run);
            if constexpr (NK == 4) {
              if (k < 8) copy(jj, k);  // step jj + 1's V pieces
            }
            // Fenced every two MFMAs (every one measured 0.4 us slower at
            // config 4: the scheduler places the pair's VALU better).
            if (k & 1) __builtin_amdgcn_sched_barrier(0);
          }
        }
        adjust(lane_max(mx), sn);
      };
      // The last iteration: tile jj's P and PV MFMAs only.
      auto last = [&](f32x16 (&sc)[2], auto par_c) {
        constexpr int P = decltype(par_c)::value;
        wait_vmcnt<0>();
        __syncthreads();
        V8 ph[2][2];
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < 8; ++i) ph[pb][h][i] = (E)__builtin_amdgcn_exp2f(sc[pb][8 * h + i]);
            l_run = sum8(ph[pb][h], l_run);
          }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int c = k & 3;
          o[k >> 2] = Op32<MODE>::mfma(vread(P, k), ph[c >> 1][c & 1], o[k >> 2]);
        }
      };
      wait_vmcnt<0>();  // the queries and step 0's K planes
      __syncthreads();
      f32x16 sA[2], sB[2];
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sA[pb][r] = negm;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          sA[pb] = Op32<MODE>::mfma(kread(0, 8 * pb + ks), qv[ks], sA[pb]);
          // Copy c: c < 2 NK the V planes of step 0, then the K planes of step 1.
          const int c = 8 * pb + ks;
          if (c < 2 * NK)
            copy_piece(c / NK, NK + c % NK);
          else if (c < 4 * NK)
            copy_piece(G + (c - 2 * NK) / NK, (c - 2 * NK) % NK);
        }
      }
      mask(0, sA);
      {
        float mx = max3f(sA[0][0], sA[0][1], sA[0][2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) mx = max3f(mx, sA[0][r], sA[0][r + 1]);
        mx = max3f(mx, sA[0][15], sA[1][0]);
#pragma unroll
        for (int r = 1; r < 15; r += 2) mx = max3f(mx, sA[1][r], sA[1][r + 1]);
        adjust(lane_max(__builtin_elementwise_maximum(mx, sA[1][15])), sA);
      }
      int j = 0;
      for (; j + 2 < steps; j += 2) {
        iter(j, sA, sB, std::integral_constant<int, 0>{});
        iter(j + 1, sB, sA, std::integral_constant<int, 1>{});
      }
      if (j + 1 < steps) {
        iter(j, sA, sB, std::integral_constant<int, 0>{});
        last(sB, std::integral_constant<int, 1>{});
      } else {
        last(sA, std::integral_constant<int, 0>{});
      }
    }
  }
  l_run = swap_sum<32>(l_run);  // the column's other half of the positions

  // The output goes through LDS (the tile ring is free once every wave is
  // past its last tile): put() writes 32 d of this lane's column, o-layout
  // o[db][4 jj + e] = O^T[32 db + 8 jj + 4 g + e][m], into region wv (16
  // KiB) as 16-byte chunks c = d / 4 of row lc, swizzled to chunk c ^ lc (the
  // 32 lanes of one chunk hit distinct banks); after a barrier, flush() has
  // every wave of the workgroup read whole rows back (group gi takes half the
  // rows of region wv), 512 contiguous bytes per half-wave, and store each
  // column's row of out with 16-byte non-temporal stores.
  static_assert(G == 2, "the two groups share the epilogue by halves");
  float* const obuf = reinterpret_cast<float*>(&lds[0][0]) + (size_t)wv * 32 * kD;
  auto put = [&](int db, const f32x16& v, float inv) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int c = 8 * db + 2 * jj + g;
      *reinterpret_cast<f32x4*>(obuf + lc * kD + 4 * (c ^ lc)) =
          f32x4{v[4 * jj] * inv, v[4 * jj + 1] * inv, v[4 * jj + 2] * inv, v[4 * jj + 3] * inv};
    }
  };
  auto flush = [&]() {
    const bool vec = aligned16(out) && q_stride % 4 == 0;
    f32x4 x[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = 4 * it + 2 * gi + g;  // row r of the region: column 32 wv + r
      x[it] = *reinterpret_cast<const f32x4*>(obuf + r * kD + 4 * (lc ^ r));
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = 4 * it + 2 * gi + g, mm = 32 * wv + r;
      if (mm % qr >= rows_here) continue;
      float* op = out + (size_t)(r0 + mm % qr) * q_stride + (size_t)(kvh * group + mm / qr) * kD + 4 * lc;
      if (vec) {
        __builtin_nontemporal_store(x[it], reinterpret_cast<f32x4*>(op));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) __builtin_nontemporal_store(x[it][e], op + e);
      }
    }
  };
  // A split's partial, laid out so a wave's stores and loads are contiguous:
  // O as 16-byte chunks c (d = 4c .. 4c + 3) of the unit's V columns,
  // chunk-major, then (max, sum) per column. Lane (lc, g) holds chunks
  // c = 8 db + 2 jj + g of its column.
  const size_t slice = (size_t)u * kv_splits;  // this unit's first split
  const size_t ml_base = (size_t)n_units * kv_splits * 32 * V;  // f32x4 units

  // The rest runs per group with its d blocks known at compile time (the
  // accumulators stay in registers). The two groups' (O, max, sum) merge by
  // halves: group GI keeps d blocks 2 GI, 2 GI + 1 of its columns and passes
  // the other two to its partner wave (same wv, other group) through the
  // upper half of the ring, (max, sum) through sm_ml; both compute the merged
  // sums with group 0's term first, so they agree to the bit, and every
  // later step (output, partial store, fold) runs on all W waves, each on
  // half of its columns' d.
  auto epilogue = [&](auto gc) {
    constexpr int GI = decltype(gc)::value, KEEP = 2 * GI, SEND = 2 - KEEP;
    __syncthreads();  // every wave is past the ring
    {
      f32x4* const xo = reinterpret_cast<f32x4*>(&lds[2][0]) + (size_t)w * 8 * 64 + lane;
#pragma unroll
      for (int bk = 0; bk < 2; ++bk)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          xo[(4 * bk + jj) * 64] = f32x4{o[SEND + bk][4 * jj], o[SEND + bk][4 * jj + 1], o[SEND + bk][4 * jj + 2],
                                         o[SEND + bk][4 * jj + 3]};
      sm_ml[w * 64 + lane] = m_run;
      sm_ml[(W + w) * 64 + lane] = l_run;
      __syncthreads();
      const int pw = (1 - GI) * VG + wv;  // partner wave
      const f32x4* const xp = reinterpret_cast<const f32x4*>(&lds[2][0]) + (size_t)pw * 8 * 64 + lane;
      const float m2 = sm_ml[pw * 64 + lane], l2 = sm_ml[(W + pw) * 64 + lane];
      const float M = fmaxf(m_run, m2);
      const float a1 = __builtin_amdgcn_exp2f(m_run - M), a2 = __builtin_amdgcn_exp2f(m2 - M);
      const float ma = GI == 0 ? a1 : a2, mb = GI == 0 ? a2 : a1;
#pragma unroll
      for (int bk = 0; bk < 2; ++bk)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 x = xp[(4 * bk + jj) * 64];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float mine = o[KEEP + bk][4 * jj + e];
            const float t0 = GI == 0 ? mine : x[e], t1 = GI == 0 ? x[e] : mine;
            o[KEEP + bk][4 * jj + e] = __builtin_fmaf(t0, ma, t1 * mb);
          }
        }
      // Written as one explicit fma so both groups round it identically.
      l_run = GI == 0 ? __builtin_fmaf(l_run, ma, l2 * mb) : __builtin_fmaf(l2, ma, l_run * mb);
      m_run = M;
    }
    if (kv_splits == 1) {
      const float inv = 1.0f / l_run;
      put(KEEP, o[KEEP], inv);
      put(KEEP + 1, o[KEEP + 1], inv);
      __syncthreads();
      flush();
      return;
    }
    {
      f32x4* ob = reinterpret_cast<f32x4*>(part) + (slice + split) * 32 * V + m;
#pragma unroll
      for (int bk = 0; bk < 2; ++bk)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          ob[(size_t)(8 * (KEEP + bk) + 2 * jj + g) * V] = f32x4{o[KEEP + bk][4 * jj], o[KEEP + bk][4 * jj + 1],
                                                                  o[KEEP + bk][4 * jj + 2], o[KEEP + bk][4 * jj + 3]};
      if (GI == 0 && g == 0)
        reinterpret_cast<float2*>(reinterpret_cast<f32x4*>(part) + ml_base)[(slice + split) * V + m] =
            float2{m_run, l_run};
    }
    // The last split to finish (its ticket the unit's last) folds the unit.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      unsigned* t = tickets + (size_t)u * 32;  // one 128-byte line per unit
      const unsigned got = __hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (got == (unsigned)kv_splits - 1) __hip_atomic_store(t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sm_ticket = got;
    }
    __syncthreads();
    if (sm_ticket != (unsigned)kv_splits - 1) return;
    // Fold in split order, the other splits' partials from this XCD's L2 and
    // this split's own from its registers (the same bits whichever split
    // finishes last: the registers hold exactly what was stored).
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(part, (short)0, (int)part_bytes, 0x00020000);
    auto o_off = [&](int sp, int c) { return (uint32_t)((((slice + sp) * 32 + c) * V + m) * 16); };
    auto ml_off = [&](int sp) { return (uint32_t)(ml_base * 16 + ((slice + sp) * V + m) * 8); };
    switch (kv_splits) {
      case 2: fold32<2, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
      case 3: fold32<3, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
      case 4: fold32<4, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
      case 5: fold32<5, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
      case 6: fold32<6, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
      case 7: fold32<7, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
      default: fold32<8, KEEP>(rs, o_off, ml_off, g, put, split, o, m_run, l_run); break;
    }
    __syncthreads();
    flush();
  };
  if (gi == 0) epilogue(std::integral_constant<int, 0>{});
  else epilogue(std::integral_constant<int, 1>{});
}

template <int S>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float* __restrict__ part, int n_rb, int n_cb,
                                                            int qr, int rows, int group, int q_stride,
                                                            float* __restrict__ out) {
  // Workgroup (kv head, row block, column block cb of 16): thread t takes
  // lane l = t % 64's chunks of d blocks t / 64 and t / 64 + 4 (1 KiB
  // contiguous per wave and split).
  const int cb = blockIdx.x % n_cb, rb = (blockIdx.x / n_cb) % n_rb, kvh = blockIdx.x / (n_cb * n_rb);
  const int l = threadIdx.x & 63, b0 = threadIdx.x >> 6;
  const int m = 16 * cb + (l & 15), kk = l >> 4;
  const int head = m / qr, row = rb * qr + m % qr;
  if (head >= group || row >= rows) return;
  const float* base = part + ((size_t)kvh * n_rb + rb) * S * kPartStride;
  f32x4 o[S][2];
  float2 ml[S];
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      o[sp][h] = reinterpret_cast<const f32x4*>(base + sp * kPartStride)[(cb * 8 + b0 + 4 * h) * 64 + l];
    ml[sp] = *reinterpret_cast<const float2*>(base + sp * kPartStride + 128 * kD + 2 * m);
  }
  float M = ml[0].x;
#pragma unroll
  for (int sp = 1; sp < S; ++sp) M = fmaxf(M, ml[sp].x);
  float L = 0.f;
  f32x4 O[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
    const float w = __builtin_amdgcn_exp2f(ml[sp].x - M);
    L += ml[sp].y * w;
#pragma unroll
    for (int h = 0; h < 2; ++h) O[h] += o[sp][h] * w;
  }
  // Non-temporal 16-byte stores where the caller's rows allow (they may be
  // only 4-byte aligned).
  float* op = out + (size_t)row * q_stride + (size_t)(kvh * group + head) * kD + 4 * kk;
  const float inv = 1.0f / L;
  const bool vec = aligned16(out) && q_stride % 4 == 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const f32x4 y = O[h] * inv;
    if (vec) {
      __builtin_nontemporal_store(y, reinterpret_cast<f32x4*>(op + 16 * (b0 + 4 * h)));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) __builtin_nontemporal_store(y[e], op + 16 * (b0 + 4 * h) + e);
    }
  }
}

struct PrefillArgs {
  const float* q;
  char* stage;
  // n_stage_tiles: a kv head's stride in the staged copy.
  int n_stage_tiles, q_stride, rows, start, group, n_rb, n_units, kv_splits;
  float qscale;
  const float* qn_w;
  float qn_eps;
  const float* qn_tab;
  float* part;
  float* out;
  TimedPair tp;
};

template <int MODE, int G, int W, int MT, int NS>
void launch_main(const PrefillArgs& a, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.n_units + 7) / 8 * 8);
  launch_timed(a.tp, prefill_kernel<MODE, G, W, MT, NS>, dim3(blocks), dim3(G * W * 64), s, a.q,
               (const char*)a.stage, a.n_stage_tiles, a.q_stride, a.rows, a.start, a.group, a.n_rb, a.n_units,
               a.kv_splits, a.qscale, a.qn_w, a.qn_eps, a.qn_tab, a.part, a.out);
}

// EXACT: one group of 4 waves with two 64 KiB stages; 128 query vectors =
// 2 column blocks per wave, 64 = 1.
void launch_exact(int vectors, const PrefillArgs& a, hipStream_t s) {
  if (vectors == 64)
    launch_main<kExact, 1, 4, 1, 2>(a, s);
  else
    launch_main<kExact, 1, 4, 2, 2>(a, s);
}

// F16 / BF16: prefill32_kernel over n_units (kv head, 256-vector block)
// units, kv_splits workgroups each.
struct P32Args {
  const float* q;
  const char* stage;
  int n_stage_tiles, q_stride, rows, start, group, n_rb, n_units, per_xcd, kv_splits;
  float qscale;
  const float* qn_w;
  float qn_eps;
  const float* qn_tab;
  const char* qprep;
  float* part;
  uint32_t part_bytes;
  unsigned* tickets;
  float* out;
  TimedPair tp;
};
template <int MODE, int W>
void launch_p32_w(const P32Args& a, hipStream_t s) {
  const unsigned blocks = (unsigned)(8 * a.per_xcd * a.kv_splits);
  launch_timed(a.tp, prefill32_kernel<MODE, W, kP32Groups>, dim3(blocks), dim3(64 * W), s, a.q, a.stage,
               a.n_stage_tiles, a.q_stride, a.rows, a.start, a.group, a.n_rb, a.n_units, a.per_xcd, a.kv_splits,
               a.qscale, a.qn_w, a.qn_eps, a.qn_tab, a.qprep, a.part, a.part_bytes, a.tickets, a.out);
}
// 128-column units on 8 waves, 64-column units on 4.
template <int MODE>
void launch_p32(int vectors, const P32Args& a, hipStream_t s) {
  if (vectors == 64)
    launch_p32_w<MODE, 4>(a, s);
  else
    launch_p32_w<MODE, kP32Waves>(a, s);
}

// Stage tiles [lo, hi) of every kv head of `layer` (positions at or past
// `positions` as zeros) into `stage`, kv heads tile_stride tiles apart.
template <int MODE, typename T>
void launch_stage_t(const T* kl, const T* vl, int n_kv, int kv_dim, int positions, int tile_stride, int lo, int hi,
                    char* stage, hipStream_t s) {
  hipLaunchKernelGGL((prefill_stage_kernel<MODE, T>), dim3((unsigned)(n_kv * (hi - lo) * 2)), dim3(kWG), 0, s, kl, vl,
                     kv_dim, positions, tile_stride, lo, hi - lo, stage);
}
template <typename T>
void launch_stage_m(uint32_t mode, const T* kl, const T* vl, int n_kv, int kv_dim, int positions, int tile_stride,
                    int lo, int hi, char* stage, hipStream_t s) {
  switch (mode) {
    case RV_PREFILL_F16: launch_stage_t<kF16, T>(kl, vl, n_kv, kv_dim, positions, tile_stride, lo, hi, stage, s); break;
    case RV_PREFILL_BF16: launch_stage_t<kBF16, T>(kl, vl, n_kv, kv_dim, positions, tile_stride, lo, hi, stage, s); break;
    default: launch_stage_t<kExact, T>(kl, vl, n_kv, kv_dim, positions, tile_stride, lo, hi, stage, s);
  }
}
void launch_stage(const rv_kv* kv, size_t layer, uint32_t mode, size_t positions, int tile_stride, int lo, int hi,
                  char* stage, hipStream_t s) {
  if (hi <= lo) return;
  const int n_kv = (int)kv->n_kv_heads, kv_dim = (int)kv->kv_dim;
  if (kv->elem == RV_ELEM_F32)
    launch_stage_m<float>(mode, (const float*)kv->k_layer(layer), (const float*)kv->v_layer(layer), n_kv, kv_dim,
                          (int)positions, tile_stride, lo, hi, stage, s);
  else
    launch_stage_m<_Float16>(mode, (const _Float16*)kv->k_layer(layer), (const _Float16*)kv->v_layer(layer), n_kv,
                             kv_dim, (int)positions, tile_stride, lo, hi, stage, s);
}

}  // namespace

size_t qprep_bytes(size_t rows, size_t n_kv_heads, size_t group, int vectors) {
  const size_t qr = vectors / group;
  return n_kv_heads * ((rows + qr - 1) / qr) * vectors * kD * 2;
}
QPrep qprep_plan(char* base, size_t rows, size_t group, float scale, int vectors) {
  const int qr = vectors / (int)group;
  return QPrep{base, (int)group, qr, (int)((rows + qr - 1) / qr), scale * kLog2e, vectors};
}
// 64-column units (4 waves, one per SIMD) where 128-column units would leave
// CUs idle and take no KV split (a short chunk on a short cache: config 3's
// 128 units become 256 workgroups and its longest unit's steps run on one
// wave per SIMD instead of two); 128 otherwise.
int prefill_vectors(const rv_kv* kv, size_t rows, size_t start, size_t group) {
  if (group == 0 || 64 % group) return kQPrepVectors;
  const long units = (long)kv->n_kv_heads * (long)((rows + kQPrepVectors / group - 1) / (kQPrepVectors / group));
  const int n_stage_tiles = (int)((start + rows + kBT - 1) / kBT);
  int kv_splits = (int)kv->tune_prefill_kv_split;
  if (kv_splits <= 0)
    kv_splits = (int)std::min<long>((kCUs + units - 1) / units, std::max(1, n_stage_tiles / (4 * kP32Groups)));
  if (!kv->xcd_ok) kv_splits = 1;
  return kv_splits <= 1 && units * 2 <= kCUs ? 64 : kQPrepVectors;
}

namespace {

int planes_of(uint32_t mode) { return (mode == RV_PREFILL_F16 || mode == RV_PREFILL_BF16) ? 1 : 2; }
// Bytes of one staged tile in `mode` (the split mode's K row exponents
// included).
size_t tile_bytes_of(uint32_t mode) {
  return planes_of(mode) == 2 ? (size_t)kTileBytes<kExact> : (size_t)kTileBytes<kF16>;
}

// The layer's persistent staged copy in `mode` (whole capacity, so tile
// addresses never move), allocated or grown on need; a change of mode or a
// new allocation marks nothing current. Sets *cap_tiles to its tile stride.
HipStatus ready_persistent(rv_kv* kv, size_t layer, uint32_t mode, hipStream_t s, int* cap_tiles) {
  HipStatus st;
  *cap_tiles = (int)((kv->capacity + kBT - 1) / kBT);
  const size_t stage_bytes = (size_t)kv->n_kv_heads * *cap_tiles * tile_bytes_of(mode);
  if (kv->staged_mode[layer] != mode || stage_bytes > kv->staged_bytes[layer]) {
    kv->staged_pos[layer] = 0;
    kv->staged_mode[layer] = mode;
  }
  if (stage_bytes > kv->staged_bytes[layer]) {
    // Never reached under capture (captured calls stage into the
    // workspace); the replaced copy is retired, not freed.
    void* p = nullptr;
    st.e = hipMalloc(&p, stage_bytes);
    if (st.e != hipSuccess) {
      st.what = "hipMalloc prefill staging";
      return st;
    }
    if (kv->staged[layer]) kv->retire(kv->staged[layer], kv->staged_bytes[layer]);
    kv->staged[layer] = p;
    kv->staged_bytes[layer] = stage_bytes;
  }
  return st;
}

}  // namespace

size_t prefill_stage_bound(const rv_kv* kv) {
  if (kv->head_dim != kD) return 0;
  const size_t cap_tiles = (kv->capacity + kBT - 1) / kBT;
  return kv->n_kv_heads * cap_tiles * tile_bytes_of(RV_PREFILL_EXACT);
}

// head_dim 128 and a group that divides 64 (so a workgroup's 64 or 128
// columns are whole rows of the group); any other geometry runs each row
// through the decode kernels.
bool prefill_supported(const rv_kv* kv, size_t group, size_t positions) {
  (void)positions;
  return kv->head_dim == kD && group >= 1 && 64 % group == 0;
}

HipStatus launch_prefill(rv_kv* kv, const float* q_rows, size_t rows, size_t n_q_heads, size_t layer,
                         size_t start, float scale, float* out, uint32_t mode, const QNorm* qn, hipStream_t s) {
  HipStatus st;
  if (rows == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const int n_kv = (int)kv->n_kv_heads;
  const uint32_t m = mode & RV_PREFILL_MODE_MASK;
  const bool split_mode = planes_of(m) == 2;
  if (split_mode && qn && qn->prepped) {
    st.e = hipErrorInvalidValue;
    st.what = "prepared queries in the split mode";
    return st;
  }
  const size_t positions = start + rows;
  const int n_stage_tiles = (int)((positions + kBT - 1) / kBT);  // tiles this call reads
  const size_t tile_bytes = tile_bytes_of(m);
  int kv_splits = (int)kv->tune_prefill_kv_split;
  int vectors, n_rb, per_xcd = 0;
  size_t part_bytes = 0;
  if (!split_mode) {
    // F16 / BF16 (prefill32_kernel): 128-column units; the KV axis is split
    // across workgroups until about kCUs of them run, each split keeping at
    // least 4 tiles of the longest block per wave group, and only where the
    // XCD fold is available.
    vectors = prefill_vectors(kv, rows, start, group);
    const int qr = vectors / group;
    n_rb = (int)((rows + qr - 1) / qr);
    const long units = (long)n_rb * n_kv;
    if (kv_splits <= 0)
      kv_splits = (int)std::min<long>((kCUs + units - 1) / units, std::max(1, n_stage_tiles / (4 * kP32Groups)));
    if (!kv->xcd_ok) kv_splits = 1;
    kv_splits = std::max(1, std::min(kv_splits, kMaxKvSplits));
    per_xcd = (int)((units + 7) / 8);
    if (kv_splits > 1) part_bytes = (size_t)units * kv_splits * vectors * kP32Part * sizeof(float);
  } else {
    // EXACT (prefill_kernel, one group of 4 waves): 128 query vectors per
    // workgroup, or 64 when 128-vector blocks would give fewer than 256
    // workgroups, but 128 when the range has at least 16 tiles, so that a KV
    // split fills the chip (config 4: 2 splits; its kernel gains more from 32
    // columns per wave than the split and merge cost: 125 vs 135 us).
    vectors = 128;
    if (kv->tune_prefill_rows > 0)
      vectors = kv->tune_prefill_rows * group <= 64 ? 64 : 128;
    else if ((long)((rows * group + 127) / 128) * n_kv < 256 && n_stage_tiles < 16)
      vectors = 64;
    const int qr = vectors / group;
    n_rb = (int)((rows + qr - 1) / qr);
    if (kv_splits <= 0) {
      // Split the KV axis until about 256 workgroups are in flight, keeping
      // at least 8 K/V tiles per split of the longest block.
      const long wgs = (long)n_rb * n_kv;
      kv_splits = (int)std::min<long>((256 + wgs - 1) / wgs, std::max<long>(1, n_stage_tiles / 8));
    }
    kv_splits = std::max(1, std::min(kv_splits, kMaxKvSplits));
    if (kv_splits > 1) part_bytes = (size_t)n_kv * n_rb * kv_splits * kPartStride * sizeof(float);
  }
  // Workspace: the split partials, then room to stage every tile this call
  // reads, which only a captured call uses; eager calls reserve it too, so
  // capturing a call of a shape already run eagerly allocates nothing.
  const size_t call_stage_bytes = (size_t)n_kv * n_stage_tiles * tile_bytes;
  // Bound for the cache's capacity: default splits keep the partials under
  // about kCUs workgroups' worth (256 rows of 128 columns in EXACT, 256
  // units of 256 columns for F16 / BF16), and a call stages at most every
  // tile of the capacity in the split mode's (largest) layout.
  const size_t bound = std::max<size_t>(part_bytes, (size_t)kCUs * kQPrepVectors * kP32Part * sizeof(float)) +
                       (size_t)n_kv * ((kv->capacity + kBT - 1) / kBT) * tile_bytes_of(RV_PREFILL_EXACT);
  st = ensure_workspace(kv, part_bytes + call_stage_bytes, bound);
  if (st.e != hipSuccess) return st;
  if (!split_mode && kv_splits > 1) {
    st = ensure_prefill_tickets(kv, (size_t)n_rb * n_kv);
    if (st.e != hipSuccess) return st;
  }
  char* stage;
  int tile_stride, stage_lo;
  float* part = (float*)kv->ws;
  if (capturing(s)) {
    // A captured graph may be replayed at any later time, so it stages
    // every tile it reads into the workspace and leaves the layer's
    // persistent copy alone.
    stage = (char*)kv->ws + part_bytes;
    tile_stride = n_stage_tiles;
    stage_lo = 0;
  } else {
    // The layer's persistent staged copy: only tiles from the first one at
    // or past its current prefix are (re)staged.
    st = ready_persistent(kv, layer, m, s, &tile_stride);
    if (st.e != hipSuccess) return st;
    size_t& staged_pos = kv->staged_pos[layer];
    stage_lo = staged_pos >= positions ? n_stage_tiles : (int)(staged_pos / kBT);
    staged_pos = std::max(staged_pos, positions);
    stage = (char*)kv->staged[layer];
  }
  launch_stage(kv, layer, m, positions, tile_stride, stage_lo, n_stage_tiles, stage, s);
  const TimedPair tp = timing_pair(kv, s);
  if (!split_mode) {
    const P32Args a{q_rows, stage, tile_stride, (int)(n_q_heads * kD), (int)rows, (int)start, group, n_rb,
                    n_rb * n_kv, per_xcd, kv_splits, scale * kLog2e, qn ? qn->w : nullptr, qn ? qn->eps : 0.f,
                    qn ? qn->tab : nullptr, qn ? qn->prepped : nullptr, part,
                    (uint32_t)std::min<size_t>(part_bytes, 0xFFFFFFF0u),
                    kv->pf_tickets, out, tp};
    if (m == RV_PREFILL_BF16)
      launch_p32<kBF16>(vectors, a, s);
    else
      launch_p32<kF16>(vectors, a, s);
  } else {
    PrefillArgs a{q_rows, stage, tile_stride, (int)(n_q_heads * kD), (int)rows,
                  (int)start, group, n_rb, n_kv * n_rb * kv_splits, kv_splits, scale * kLog2e,
                  qn ? qn->w : nullptr, qn ? qn->eps : 0.f, qn ? qn->tab : nullptr, part, out, tp};
    launch_exact(vectors, a, s);
    if (kv_splits > 1) {
      const int qr = vectors / group;
      const dim3 grid((unsigned)(n_kv * n_rb * vectors / 16));
      const int n_cb = vectors / 16, q_stride = (int)(n_q_heads * kD);
#define RV_MERGE(S)                                                                                               \
  case S:                                                                                                         \
    hipLaunchKernelGGL(prefill_merge_kernel<S>, grid, dim3(256), 0, s, (const float*)part, n_rb, n_cb, qr, (int)rows, \
                       group, q_stride, out);                                                                    \
    break
      switch (kv_splits) {
        RV_MERGE(2);
        RV_MERGE(3);
        RV_MERGE(4);
        RV_MERGE(5);
        RV_MERGE(6);
        RV_MERGE(7);
        default: RV_MERGE(8);
      }
#undef RV_MERGE
    }
  }
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "prefill launch";
  return st;
}

// The F16 / BF16 fold's ticket lines (one 128-byte line per unit), grown on
// need outside capture, zeroed when allocated; every call's last split resets
// its unit's counter, so they stay zero between calls.
HipStatus ensure_prefill_tickets(rv_kv* kv, size_t units) {
  HipStatus st;
  if (units <= kv->pf_ticket_units) return st;
  if (capturing(kv->stream)) {
    st.e = hipErrorStreamCaptureUnsupported;
    st.what = "prefill ticket growth under graph capture (run a call of this shape uncaptured first)";
    return st;
  }
  const size_t want = std::max<size_t>(units, 1024);
  void* p = nullptr;
  st.e = hipMalloc(&p, want * 128);
  if (st.e == hipSuccess) st.e = hipMemset(p, 0, want * 128);
  if (st.e == hipSuccess) st.e = hipDeviceSynchronize();
  if (st.e != hipSuccess) {
    if (p) (void)hipFree(p);
    st.what = "hipMalloc prefill tickets";
    return st;
  }
  if (kv->pf_tickets) kv->retire(kv->pf_tickets, kv->pf_ticket_units * 128);
  kv->pf_tickets = (unsigned*)p;
  kv->pf_ticket_units = want;
  return st;
}

HipStatus prepare_prefill_stage(rv_kv* kv, size_t layer, size_t pos0, size_t rows, uint32_t mode,
                                hipStream_t s, StageDst* sd) {
  HipStatus st;
  *sd = StageDst{};
  const uint32_t m = mode & RV_PREFILL_MODE_MASK;
  // Split-mode tiles carry exponents over all of their rows, which rows
  // appended one at a time would change: the attention call's stage kernel
  // converts them from the cache instead.
  if (rows == 0 || kv->head_dim != kD || capturing(s) || planes_of(m) == 2) return st;
  int tile_stride;
  st = ready_persistent(kv, layer, m, s, &tile_stride);
  if (st.e != hipSuccess) return st;
  size_t& staged_pos = kv->staged_pos[layer];
  // Rows below pos0 not yet current (decode steps, plain appends, a new
  // mode): staged from the cache, their last tile zero-filled from pos0 on,
  // which the chunk's rows then overwrite.
  if (staged_pos < pos0)
    launch_stage(kv, layer, m, pos0, tile_stride, (int)(staged_pos / kBT), (int)((pos0 + kBT - 1) / kBT),
                 (char*)kv->staged[layer], s);
  staged_pos = pos0 + rows;
  sd->base = (char*)kv->staged[layer];
  sd->tile_stride = tile_stride;
  sd->mode = m;
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "prefill stage launch";
  return st;
}

}  // namespace rv
