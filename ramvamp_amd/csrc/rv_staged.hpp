// rv_staged.hpp — the staged K/V tile layout that the prefill attention
// kernels read, shared by the kernels that write it: the prefill stage
// kernel (converting cache rows) and the row prologue (writing a prefill
// chunk's own rows as it appends them).
#pragma once

#include "rv_device.hpp"

namespace rv {

constexpr int kBT = 64;             // positions per K/V tile
constexpr int kPlaneBytes = 16384;  // one staged 64 x 128 plane of 2-byte elements

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// Arithmetic modes of the staged copy (RV_PREFILL_EXACT / F16 / BF16).
enum Mode { kExact = 0, kF16 = 1, kBF16 = 2 };

template <int MODE>
struct Op;
template <>
struct Op<kExact> {
  typedef _Float16 E;
  typedef f16x8 V8;
  typedef f16x4 V4;
  static constexpr bool kSplit = true;
  __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <>
struct Op<kF16> {
  typedef _Float16 E;
  typedef f16x8 V8;
  typedef f16x4 V4;
  static constexpr bool kSplit = false;
  __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <>
struct Op<kBF16> {
  typedef __bf16 E;
  typedef bf16x8 V8;
  typedef bf16x4 V4;
  static constexpr bool kSplit = false;
  __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

// Planes per K or V half of a staged tile: hi and lo in the split mode.
template <int MODE>
constexpr int kPlanes = Op<MODE>::kSplit ? 2 : 1;

// The split mode keeps any finite fp32 K and V in f16 hi + lo planes by
// scaling with powers of two: each K row t by its exponent e_t, each V
// column d of a tile by its exponent c_d (so a tile's exponents depend on all
// of its rows, and only the stage kernel, converting whole tiles from the
// cache, writes split-mode tiles). The tile ends with a 4 KiB region of
// 1 KiB pieces holding the factors that undo the scaling, as floats: 2^-e_t
// at byte kScaleOffset + 4 t (the first piece), 2^-c_d at byte
// kVScaleOffset + 4 d (the second), two unused, so the K half of a tile (its
// planes and factors) and the V half can be copied into LDS separately.
constexpr int kScaleBytes = 4096;
constexpr int kScaleOffset = 4 * kPlaneBytes;
constexpr int kVScaleOffset = kScaleOffset + 1024;
template <int MODE>
constexpr int kTileBytes = 2 * kPlanes<MODE> * kPlaneBytes + (Op<MODE>::kSplit ? kScaleBytes : 0);

// The power-of-two exponent e that puts amax * 2^e in [2^13, 2^14), at most
// cap, or 0 for a zero or non-finite amax (such a row is staged as it is).
// The default cap keeps 2^-e a float (2^-149 is its smallest subnormal); a
// capped vector, all of whose elements are below 2^-135, is scaled to
// magnitudes in [1, 2^14), inside f16's normal range.
__device__ __forceinline__ int scale_exponent(float amax, int cap = 149) {
  if (!(amax > 0.f) || !__builtin_isfinite(amax)) return 0;
  return min(14 - __builtin_amdgcn_frexp_expf(amax), cap);
}

// hi = round(x); lo = round(x - hi), into element e of two vectors.
template <typename E, typename V>
__device__ __forceinline__ void split2v(float x, V& hi, V& lo, int e) {
  const E h = (E)x;
  hi[e] = h;
  lo[e] = (E)(x - (float)h);
}

// ---- staged tile layout -------------------------------------------------------------
// One tile = P planes of K, then P planes of V^T (P = 2 in the split mode:
// hi, lo; then the split mode's exponent region), each plane 16 KiB of
// 16-byte chunks (8 elements).
//   K plane: row t (64) x chunk c (16): elements d = 8c .. 8c+7, stored at
//     byte 256 t + 16 (c ^ (t & 15)).
//   V^T plane: row d (128) x chunk c (8), stored at byte
//     128 d + 16 (c ^ ((d >> 1) & 7)); which positions a chunk holds follows
//     the order the mode's attention kernel produces P in (vt_pos_m):
//     the split mode (16x16 MFMA tiles): chunk c = 4 s2 + k holds, in slot
//       j, position t = 32 s2 + 4k + j (j < 4) or 32 s2 + 16 + 4k + j - 4
//       (j >= 4);
//     F16 / BF16 (32x32 MFMA tiles): chunk c = 4 pb + 2 h + g holds, in
//       slot j, position t = 32 pb + 16 h + 4 g + 8 (j / 4) + j % 4.
//   In both, positions 4i .. 4i + 3 fill 8 contiguous bytes of one chunk.
// The swizzles put the 16 lanes of one operand read on 16 distinct 16-byte
// bank groups; the counters read no LDS bank conflicts for either plane
// (an alternative V^T layout with each 32-position half contiguous,
// 8192 s2 + 64 d + 16 (k ^ ((d >> 2) & 3)), read ~4 conflict cycles per
// operand read).
__device__ __forceinline__ int k_off(int t, int c) { return 256 * t + 16 * (c ^ (t & 15)); }
__device__ __forceinline__ int vt_off(int d, int c) { return 128 * d + 16 * (c ^ ((d >> 1) & 7)); }
__device__ __forceinline__ int vt_pos(int c, int j) {
  const int s2 = c >> 2, k = c & 3;
  return j < 4 ? 32 * s2 + 4 * k + j : 32 * s2 + 16 + 4 * k + (j - 4);
}
// Byte of element (position t, dim d) in a V^T plane: the inverse of vt_pos
// (t = 32 s2 + u: chunk 4 s2 + (u & 15) / 4, slot (u & 3) + 4 (u >= 16)).
__device__ __forceinline__ int vt_byte(int d, int t) {
  const int u = t & 31;
  return vt_off(d, 4 * (t >> 5) + ((u & 15) >> 2)) + 2 * ((u & 3) + ((u >> 4) << 2));
}
// The F16 / BF16 map: chunk 4 pb + 2 h + g, slot 4 (w / 8) + w % 4 for
// t = 32 pb + 16 h + w, g = (w / 4) % 2.
__device__ __forceinline__ int vt_pos32(int c, int j) {
  return 32 * (c >> 2) + 16 * ((c >> 1) & 1) + 4 * (c & 1) + 8 * (j >> 2) + (j & 3);
}
__device__ __forceinline__ int vt_byte32(int d, int t) {
  const int w = t & 15;
  return vt_off(d, 4 * (t >> 5) + 2 * ((t >> 4) & 1) + ((w >> 2) & 1)) + 2 * (4 * (w >> 3) + (w & 3));
}
template <int MODE>
__device__ __forceinline__ int vt_pos_m(int c, int j) {
  return Op<MODE>::kSplit ? vt_pos(c, j) : vt_pos32(c, j);
}
template <int MODE>
__device__ __forceinline__ int vt_byte_m(int d, int t) {
  return Op<MODE>::kSplit ? vt_byte(d, t) : vt_byte32(d, t);
}

// Eight consecutive floats: two 16-byte loads when `vec` (p 16-byte
// aligned), else eight 4-byte loads.
__device__ __forceinline__ void ld8(const float* p, bool vec, float (&o)[8]) {
  if (vec) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = a[e];
      o[4 + e] = b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = p[e];
  }
}

__device__ __forceinline__ bool aligned16(const void* a, const void* b = nullptr, const void* c = nullptr) {
  return (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15) == 0;
}

// This lane's 64 elements of one query vector, x[ks][i] = q[16 ks + 8 g + i]
// (its partner lane, 32 apart, holds the other 64), with the q prologue's
// operands when qn_w is given: the loads only (Q32Loads::issue), so the
// caller can queue the first tiles' loads behind them before anything
// waits, then the prologue (finish): RMSNorm with an f64 sum of squares over
// the pair, then `x * inv * w` and the rotation of the pairs (d, d + 64)
// (both in this lane: ks and ks + 4), in the reference's separately rounded
// f32 operations, with the row's (cos, sin) from tab_row (64 cos, then 64
// sin), as the row prologue would.
struct Q32Loads {
  float x[8][8];
  float w0[4][8], w1[4][8], cs[4][8], sn[4][8];
  __device__ __forceinline__ void issue(const float* qp, int g, const float* __restrict__ qn_w,
                                        const float* __restrict__ tab_row) {
    const bool vec = aligned16(qp, qn_w, tab_row);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) ld8(qp + 16 * ks + 8 * g, vec, x[ks]);
    if (!qn_w) return;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int i = 16 * ks + 8 * g;
      ld8(qn_w + i, vec, w0[ks]);
      ld8(qn_w + i + 64, vec, w1[ks]);
      ld8(tab_row + i, vec, cs[ks]);
      ld8(tab_row + 64 + i, vec, sn[ks]);
    }
  }
  __device__ __forceinline__ void finish(bool norm, float qn_eps) {
#pragma clang fp contract(off)
    if (!norm) return;
    double ss = 0.0;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (double)x[ks][e] * (double)x[ks][e];
    ss = swap_sum_f64<32>(ss);
    const float inv = (float)(1.0 / sqrt(ss / 128.0 + (double)qn_eps));  // head_dim 128
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a0 = x[ks][e] * inv * w0[ks][e], a1 = x[ks + 4][e] * inv * w1[ks][e];
        x[ks][e] = a0 * cs[ks][e] - a1 * sn[ks][e];
        x[ks + 4][e] = a0 * sn[ks][e] + a1 * cs[ks][e];
      }
  }
};

// Prepared queries of the F16 / BF16 prefill: a chunk's row prologue writes
// each query head's row after RMSNorm and RoPE, times log2(e) * scale,
// rounded to the MFMA type, straight into the attention kernel's operand
// order, so that kernel's query loads are eight coalesced 16-byte loads per
// lane. The kernel's units (kv head * n_rb + rb) hold V = 128 (kQPrepVectors)
// or 64 columns each (prefill_vectors): column m of unit u is query head kv head * group + m / qr of
// row rb * qr + m % qr (qr = V / group), global column c = u * V + m. Element d
// of column c sits in 16-byte chunk ((c / 32) * 8 + d / 16) * 64 + 32 * ((d /
// 8) & 1) + c % 32 at position d % 8: the B operand (Q^T) of the QK step
// d / 16 of the wave owning columns c - c % 32 .. + 31, in lane order.
constexpr int kQPrepVectors = 128;
__host__ __device__ inline size_t qprep_index(size_t c, int d) {
  return ((((c >> 5) * 8 + (size_t)(d >> 4)) * 64 + 32 * ((d >> 3) & 1) + (c & 31)) * 8 + (d & 7));
}

}  // namespace rv
