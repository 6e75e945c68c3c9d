// rv_quant.hip — the quantized projections either side of attention on gfx950:
// Q8_K / Q8_0 activation quantizers and the k-quant / Q8_0 GEMVs.
//
// Replaces quantize_row_q8_k / quantize_row_q8_0
// (crates/core/src/kernels/quants/quantize.rs:37-106) and the row-range GEMVs
// gemv_q8_k_rows / gemv_q8_0_rows (kernels/gemv.rs:296-615) over the scalar
// dots vec_dot_{q4_k,q5_k,q6_k}_q8_k / vec_dot_q8_0_q8_0 (quants/dot.rs),
// as called at model/forward.rs:2574-2646.
//
// Results are bit-identical to the reference's scalar kernels:
//  - quantizers: one wave per 256-value Q8_K block (the first value of
//    largest magnitude found by a lane-ordered wave reduction, RNE rounding,
//    the scalar code's f32 divisions) and 32 lanes per Q8_0 block;
//  - GEMVs: one wave per output row. Lanes split each super-block's
//    sub-blocks and form the integer sub-block sums with v_dot4_i32_i8
//    (exact, in any order), a block's integer totals come from an exact
//    8-lane reduction, the block's float contribution is the scalar dot's
//    expression, and the row's sum adds the blocks in order.
// The GEMVs stream each weight byte once (HBM-bound); activations are
// re-read per row from L2.
#include "rv_device.hpp"
#include "rv_internal.hpp"
#include "rv_quant.hpp"

namespace rv {
namespace {

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

// 32 bytes at a 2-byte-aligned address, as 8 little-endian dwords, reading
// nothing outside [a, a + 32) except the two bytes before `a` (which the
// callers' layouts guarantee belong to the same block).
__device__ __forceinline__ void load32_a2(const uint8_t* a, uint32_t (&w)[8]) {
  if (((uintptr_t)a & 2) == 0) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(a);
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = p[k];
    return;
  }
  const uint32_t* p = reinterpret_cast<const uint32_t*>(a - 2);  // bytes a-2 .. a+1
  uint32_t e[8];
#pragma unroll
  for (int k = 0; k < 7; ++k) e[k + 1] = p[k + 1];  // bytes a+2+4k .. a+5+4k
  e[0] = p[0];
  const uint32_t tail = *reinterpret_cast<const uint16_t*>(a + 30);
#pragma unroll
  for (int k = 0; k < 7; ++k) w[k] = __builtin_amdgcn_alignbyte(e[k + 1], e[k], 2);
  w[7] = (e[7] >> 16) | (tail << 16);
}

// Sum over the 8 lanes of an aligned lane group (exact for integers).
__device__ __forceinline__ int sum8_lanes(int v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  return v;
}

__device__ __forceinline__ int dot4(uint32_t w, int a, int acc) {
  return __builtin_amdgcn_sdot4((int)w, a, acc, false);
}

__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// get_scale_min_k4 (quants/blocks.rs:158-167) from the 12 scale bytes as
// three little-endian dwords.
__device__ __forceinline__ void scale_min_k4(int j, const uint32_t (&s)[3], int& sc, int& m) {
  auto byte = [&](int i) { return (int)((s[i >> 2] >> (8 * (i & 3))) & 0xFF); };
  if (j < 4) {
    sc = byte(j) & 63;
    m = byte(j + 4) & 63;
  } else {
    sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
    m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// 16 bytes at a 4-byte-aligned global address (global_load_dwordx4 needs
// only dword alignment).
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

// Lane j's view of one Q8_K activation block: qs[32j .. 32j+31] packed 4
// per int, the scale d, and bsums[2j], bsums[2j+1].
struct ActK {
  int a[8];
  float d;
  int bs_lo, bs_hi;
};

__device__ __forceinline__ ActK act_from_block(const rv_block_q8_k* __restrict__ y, int j) {
  ActK r;
  const int* q = reinterpret_cast<const int*>(y->qs + 32 * j);
#pragma unroll
  for (int k = 0; k < 8; ++k) r.a[k] = q[k];
  const uint32_t bs = *reinterpret_cast<const uint32_t*>(y->bsums + 2 * j);
  r.bs_lo = (int)(int16_t)(bs & 0xFFFFu);
  r.bs_hi = (int)(int16_t)(bs >> 16);
  r.d = y->d;
  return r;
}

// One super-block's float contribution for the k-quants, computed by the 8
// lanes of a group, lane j owning sub-block j (Q4_K/Q5_K: 32 weights) or
// the two 16-weight sub-blocks 2j, 2j+1 (Q6_K); every lane of the group
// returns the same value.
template <int FMT>
__device__ __forceinline__ float kq_block(const uint8_t* __restrict__ blk, const ActK& y, int j);

// k_quant_affine_block with the q4_K / q5_K expansions (dot.rs:56-143):
// d*sumi - dmin*sumi_mins, d = f16(d)*y.d, dmin = f16(dmin)*y.d.
template <int FMT>
__device__ __forceinline__ float affine_block(const uint8_t* __restrict__ blk, const ActK& y, int j) {
#pragma clang fp contract(off)
  constexpr bool kQ5 = FMT == RV_QF_Q5_K;
  const uint32_t dd = *reinterpret_cast<const uint32_t*>(blk);
  const uint32_t* sp = reinterpret_cast<const uint32_t*>(blk + 4);
  const uint32_t s[3] = {sp[0], sp[1], sp[2]};
  const u32x4a* qp = reinterpret_cast<const u32x4a*>(blk + (kQ5 ? 48 : 16) + 32 * (j >> 1));
  const u32x4a q0 = qp[0], q1 = qp[1];
  const uint32_t q[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
  uint32_t qh[8];
  if constexpr (kQ5) {
    const u32x4a* hp = reinterpret_cast<const u32x4a*>(blk + 16);
    const u32x4a h0 = hp[0], h1 = hp[1];
    qh[0] = h0[0], qh[1] = h0[1], qh[2] = h0[2], qh[3] = h0[3];
    qh[4] = h1[0], qh[5] = h1[1], qh[6] = h1[2], qh[7] = h1[3];
  }
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t w = (j & 1) ? (q[k] >> 4) & 0x0F0F0F0Fu : q[k] & 0x0F0F0F0Fu;
    if constexpr (kQ5) w |= ((qh[k] >> j) & 0x01010101u) << 4;
    acc = dot4(w, y.a[k], acc);
  }
  int sc, m;
  scale_min_k4(j, s, sc, m);
  const int sumi = sum8_lanes(sc * acc);
  const int sumi_mins = sum8_lanes(m * (y.bs_lo + y.bs_hi));
  const float d = f16_bits_to_f32(dd) * y.d;
  const float dmin = f16_bits_to_f32(dd >> 16) * y.d;
  return d * (float)sumi - dmin * (float)sumi_mins;
}

template <>
__device__ __forceinline__ float kq_block<RV_QF_Q4_K>(const uint8_t* blk, const ActK& y, int j) {
  return affine_block<RV_QF_Q4_K>(blk, y, j);
}
template <>
__device__ __forceinline__ float kq_block<RV_QF_Q5_K>(const uint8_t* blk, const ActK& y, int j) {
  return affine_block<RV_QF_Q5_K>(blk, y, j);
}

// vec_dot_q6_k_q8_k (dot.rs:150-179): lane j = 4 half + group holds weights
// 32j .. 32j+31: ql nibbles (byte l + 32 (group & 1) of the half, high
// nibble for groups 2, 3) and two qh bits (2 group). The stored values are
// q + 32 in 0..63; sum (q+32)a - 32 sum a, with sum a the activation bsums.
template <>
__device__ __forceinline__ float kq_block<RV_QF_Q6_K>(const uint8_t* blk, const ActK& y, int j) {
#pragma clang fp contract(off)
  const int half = j >> 2, grp = j & 3;
  uint32_t ql[8], qh[8];
  load32_a2(blk + 64 * half + 32 * (grp & 1), ql);
  load32_a2(blk + 128 + 32 * half, qh);
  int lo = 0, hi = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t nib = (grp >> 1) ? (ql[k] >> 4) & 0x0F0F0F0Fu : ql[k] & 0x0F0F0F0Fu;
    const uint32_t w = nib | (((qh[k] >> (2 * grp)) & 0x03030303u) << 4);
    if (k < 4)
      lo = dot4(w, y.a[k], lo);
    else
      hi = dot4(w, y.a[k], hi);
  }
  lo -= 32 * y.bs_lo;
  hi -= 32 * y.bs_hi;
  const uint32_t scp = *reinterpret_cast<const uint16_t*>(blk + 192 + 2 * j);
  const int sc_lo = (int)(int8_t)(scp & 0xFF), sc_hi = (int)(int8_t)(scp >> 8);
  const int sumi = sum8_lanes(sc_lo * lo + sc_hi * hi);
  const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 208));
  return d * y.d * (float)sumi;
}

// One k-quant row against its Q8_K activation blocks (global memory or
// LDS), every lane returning the row's sum: 8 super-blocks per pass (lane
// group b), added in block order.
template <int FMT>
__device__ __forceinline__ float kq_row(const uint8_t* __restrict__ row, int nb, const rv_block_q8_k* __restrict__ acts,
                                        int lane) {
  constexpr int BB = FMT == RV_QF_Q4_K ? 144 : FMT == RV_QF_Q5_K ? 176 : 210;
  const int bl = lane >> 3, j = lane & 7;
  float sumf = 0.f;
  for (int b0 = 0; b0 < nb; b0 += 8) {
    const int b = min(b0 + bl, nb - 1);  // groups past the row recompute its last block (unused)
    const float c = kq_block<FMT>(row + (size_t)b * BB, act_from_block(acts + b, j), j);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (b0 + k < nb) sumf += lane_f(c, 8 * k);
  }
  return sumf;
}

// vec_dot_q8_0_q8_0 (dot.rs:185-201): lane per 32-weight block, 64 blocks
// per pass, sumf += sumi * (f16(d) * y.d) in block order.
__device__ __forceinline__ float q80_row(const uint8_t* __restrict__ row, int nb, const rv_block_q8_0* __restrict__ acts,
                                         int lane) {
#pragma clang fp contract(off)
  float sumf = 0.f;
  for (int b0 = 0; b0 < nb; b0 += 64) {
    const int b = min(b0 + lane, nb - 1);
    const uint8_t* blk = row + (size_t)b * 34;
    uint32_t w[8];
    load32_a2(blk + 2, w);
    const int* a = reinterpret_cast<const int*>(acts[b].qs);
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) s = dot4(w[k], a[k], s);
    const float c = (float)s * (f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk)) * acts[b].d);
    const int n = min(64, nb - b0);
    for (int k = 0; k < n; ++k) sumf += lane_f(c, k);
  }
  return sumf;
}

// quantize_row_q8_k (quantize.rs:71-106) of one block by one wave, lane l
// holding values 4l .. 4l+3: the first value of largest magnitude (per lane
// in order, then across lanes by magnitude and lowest index; magnitudes of
// 0 and NaN never win, as `av > amax` from amax = 0 never takes them), RNE
// rounding, the clamp, bsums, and the scalar code's f32 divisions.
__device__ __forceinline__ void quantize_block_q8_k(const float* __restrict__ xs, rv_block_q8_k* blk, int lane) {
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = xs[4 * lane + e];
  float amax = 0.f, mx = 0.f;
  int idx = 1 << 30;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float av = fabsf(v[e]);
    if (av > amax) {
      amax = av;
      mx = v[e];
      idx = 4 * lane + e;
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float a2 = __shfl_xor(amax, off, 64), m2 = __shfl_xor(mx, off, 64);
    const int i2 = __shfl_xor(idx, off, 64);
    if (a2 > amax || (a2 == amax && i2 < idx)) {
      amax = a2;
      mx = m2;
      idx = i2;
    }
  }
  if (amax == 0.f) {  // wave-uniform
    *reinterpret_cast<uint32_t*>(blk->qs + 4 * lane) = 0u;
    if (lane < 16) blk->bsums[lane] = 0;
    if (lane == 0) blk->d = 0.f;
    return;
  }
  const float iscale = -127.f / mx;
  uint32_t packed = 0;
  int gsum = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int n = min(max((int)__builtin_rintf(iscale * v[e]), -128), 127);
    packed |= (uint32_t)(n & 0xFF) << (8 * e);
    gsum += n;
  }
  *reinterpret_cast<uint32_t*>(blk->qs + 4 * lane) = packed;
  // bsums[g]: the 16 values of lanes 4g .. 4g+3.
  gsum += __shfl_xor(gsum, 1, 64);
  gsum += __shfl_xor(gsum, 2, 64);
  if ((lane & 3) == 0) blk->bsums[lane >> 2] = (int16_t)gsum;
  if (lane == 0) blk->d = 1.f / iscale;
}

// quantize_row_q8_0 (quantize.rs:37-55) of one block by the 32 lanes of a
// half-wave, lane i holding value i: d = amax/127, q = round(v/d) half away
// from zero, d stored f16-rounded.
__device__ __forceinline__ void quantize_block_q8_0(const float* __restrict__ xs, rv_block_q8_0* blk, int i) {
  const float v = xs[i];
  float amax = fabsf(v);
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float d = amax / 127.f;
  const float id = d != 0.f ? 1.f / d : 0.f;
  blk->qs[i] = (int8_t)roundf(v * id);
  if (i == 0) blk->d = (float)(_Float16)d;
}

__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float* __restrict__ x, rv_block_q8_k* __restrict__ out,
                                                           int n_blocks) {
  const int b = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= n_blocks) return;  // wave-uniform
  quantize_block_q8_k(x + (size_t)b * 256, out + b, threadIdx.x & 63);
}

__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ x, rv_block_q8_0* __restrict__ out,
                                                           int n_blocks) {
  const int t = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const int b = t >> 5;
  if (b >= n_blocks) return;  // whole 32-lane halves
  quantize_block_q8_0(x + (size_t)b * 32, out + b, t & 31);
}

// Both forms in one launch: wave b quantizes 256-value block b to Q8_K and
// its eight 32-value blocks to Q8_0 (each half-wave four of them), with the
// same per-block code as the two kernels above, so the same bytes.
__global__ __launch_bounds__(256) void quantize_both_kernel(const float* __restrict__ x, rv_block_q8_k* __restrict__ ok,
                                                            rv_block_q8_0* __restrict__ o0, int n_blocks) {
  const int b = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= n_blocks) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const float* xb = x + (size_t)b * 256;
  quantize_block_q8_k(xb, ok + b, lane);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sb = 2 * i + (lane >> 5);
    quantize_block_q8_0(xb + 32 * sb, o0 + (size_t)b * 8 + sb, lane & 31);
  }
}

__device__ __forceinline__ float row_dot(uint32_t fmt, const uint8_t* row, int nb, const void* acts, int lane) {
  switch (fmt) {
    case RV_QF_Q4_K: return kq_row<RV_QF_Q4_K>(row, nb, (const rv_block_q8_k*)acts, lane);
    case RV_QF_Q5_K: return kq_row<RV_QF_Q5_K>(row, nb, (const rv_block_q8_k*)acts, lane);
    case RV_QF_Q6_K: return kq_row<RV_QF_Q6_K>(row, nb, (const rv_block_q8_k*)acts, lane);
    default: return q80_row(row, nb, (const rv_block_q8_0*)acts, lane);
  }
}

constexpr int kRowsPerWG = 4;

// out[i] = row(row_lo + i) . acts for i < n_rows, acts quantized blocks in
// global memory; one wave per row.
template <int FMT>
__global__ __launch_bounds__(64 * kRowsPerWG) void gemv_rows_kernel(const uint8_t* __restrict__ w, size_t row_bytes,
                                                                    int nb, const void* __restrict__ acts, long row_lo,
                                                                    int n_rows, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int i = (int)blockIdx.x * kRowsPerWG + (threadIdx.x >> 6);
  if (i >= n_rows) return;  // wave-uniform
  const uint8_t* row = w + (size_t)(row_lo + i) * row_bytes;
  float v;
  if constexpr (FMT == RV_QF_Q8_0)
    v = q80_row(row, nb, (const rv_block_q8_0*)acts, lane);
  else
    v = kq_row<FMT>(row, nb, (const rv_block_q8_k*)acts, lane);
  if (lane == 0) out[i] = v;
}

// The fused projections: one row per wave, 8 waves per workgroup, the f32
// activation row quantized once per workgroup into LDS first (the same
// per-block code as the quantizer kernels, so bit-identical), then every
// wave's GEMV row reads its blocks from LDS. Segments (at most 3) are row
// ranges of independent matrices, each against the Q8_K or the Q8_0 form.
// 1 / sqrt(mean(x^2) + eps) of n values, as norm.rs:18-26 computes it: the
// squares summed in f64 (here per thread, then over lanes and waves in a
// fixed order, so every thread of the workgroup gets the same value), sqrt
// and reciprocal in f64, rounded once to f32. `red` holds NT / 64 doubles.
template <int NT>
__device__ __forceinline__ float block_inv_rms(const float* __restrict__ x, int n, float eps, double* red) {
  double ss = 0.0;
  for (int i = threadIdx.x; i < n; i += NT) {
    const double v = (double)x[i];
    ss += v * v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) tot += red[w];
  return (float)(1.0 / sqrt(tot / (double)n + (double)eps));
}

template <bool NORM>
__global__ __launch_bounds__(64 * kFusedWaves) void fused_proj_kernel(FusedProjArgs a) {
  __shared__ rv_block_q8_k lk[kFusedMaxKBlocks];
  __shared__ rv_block_q8_0 l0[kFusedMax0Blocks];
  // The wave index as a scalar: the row, its segment and the segment's
  // fields are then wave-uniform, read with scalar loads from the kernel
  // arguments (indexed from a vector register, each was a vector load of
  // the argument segment that every later load waited behind).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (a.gate_pos && *a.gate_pos > a.gate_max) return;  // the whole grid: its decode step was refused
  const int first = (int)blockIdx.x * kFusedWaves;
  // The segments this workgroup's rows touch decide which forms it needs.
  bool need_k = false, need_0 = false;
  {
    int lo = 0;
    for (int sg = 0; sg < a.n_seg; ++sg) {
      const int hi = lo + a.n_rows[sg];
      if (first < hi && first + kFusedWaves > lo) (a.seg[sg].fmt == RV_QF_Q8_0 ? need_0 : need_k) = true;
      lo = hi;
    }
  }
  int i = first + wave, sg = 0;
  while (sg < a.n_seg && i >= a.n_rows[sg]) i -= a.n_rows[sg++];
  // This wave's weight row starts streaming while the workgroup quantizes:
  // one dword from each of its 128-byte lines (lane l: byte 128 l, clamped
  // to the row and aligned down; the matrix base is 4-byte aligned, so the
  // address stays inside it). The value is consumed only after the barrier,
  // so nothing waits for it. With the norm it is issued after the loads of
  // x and the norm weight, which the norm waits for first (loads retire in
  // order).
  uint32_t touch = 0;
  auto touch_row = [&]() {
    if (sg < a.n_seg) {
      const FusedSeg& s = a.seg[sg];
      const uint8_t* row = s.w + (size_t)i * s.row_bytes;
      const size_t off = min((size_t)128 * lane, s.row_bytes - 4);
      touch = *reinterpret_cast<const uint32_t*>((uintptr_t)(row + off) & ~(uintptr_t)3);
    }
  };
  if constexpr (!NORM) touch_row();
  // The residual an output row is added to is read now, under the rest.
  float addv = 0.f;
  if (sg < a.n_seg && a.seg[sg].add && lane == 0) addv = a.seg[sg].add[i];
  const float* x = a.x;
  if constexpr (NORM) {
#pragma clang fp contract(off)
    // The normalized row, x * inv * w left to right in f32 (norm.rs:55-57),
    // staged in LDS for the quantizers. Each thread loads its values of x
    // and w once (x <= 8192 values: at most 16 per thread), so the sum of
    // squares and the scaling cost one memory round trip between them.
    constexpr int NT = 64 * kFusedWaves, PER = kFusedMaxKBlocks * 256 / NT;
    __shared__ float xs[kFusedMaxKBlocks * 256];
    __shared__ double red[kFusedWaves];
    const int n = a.nbk * 256;
    float xr[PER], wr[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int j = threadIdx.x + r * NT;
      xr[r] = j < n ? a.x[j] : 0.f;
      wr[r] = j < n ? a.norm_w[j] : 0.f;
    }
    asm volatile("" ::: "memory");  // the row loads above issue first
    touch_row();
    double ss = 0.0;
#pragma unroll
    for (int r = 0; r < PER; ++r) ss += (double)xr[r] * (double)xr[r];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < kFusedWaves; ++w) tot += red[w];
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)a.eps));
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int j = threadIdx.x + r * NT;
      if (j < n) xs[j] = xr[r] * inv * wr[r];
    }
    __syncthreads();
    x = xs;
  }
  if (need_k)
    for (int b = wave; b < a.nbk; b += kFusedWaves) quantize_block_q8_k(x + (size_t)b * 256, &lk[b], lane);
  if (need_0)
    for (int b = 2 * wave + (lane >> 5); b < a.nb0; b += 2 * kFusedWaves)
      quantize_block_q8_0(x + (size_t)b * 32, &l0[b], lane & 31);
  __syncthreads();
  asm volatile("" ::"v"(touch));
  if (sg >= a.n_seg) return;  // wave-uniform
  const FusedSeg& s = a.seg[sg];
  const bool q80 = s.fmt == RV_QF_Q8_0;
  const float v = row_dot(s.fmt, s.w + (size_t)i * s.row_bytes, q80 ? a.nb0 : a.nbk,
                          q80 ? (const void*)l0 : (const void*)lk, lane);
  if (lane == 0) s.out[i] = s.add ? addv + v : v;
}

__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float eps, int n, float* __restrict__ out) {
  __shared__ double red[16];
  const float inv = block_inv_rms<1024>(x, n, eps, red);
  for (int j = threadIdx.x; j < n; j += 1024) {
#pragma clang fp contract(off)
    out[j] = x[j] * inv * w[j];
  }
}

// One workgroup per row: out[r] = rmsnorm(x[r], w, eps) over n values.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float eps, int n, float* __restrict__ out) {
  __shared__ double red[4];
  const float* xr = x + (size_t)blockIdx.x * n;
  float* orow = out + (size_t)blockIdx.x * n;
  const float inv = block_inv_rms<256>(xr, n, eps, red);
  for (int j = threadIdx.x; j < n; j += 256) {
#pragma clang fp contract(off)
    orow[j] = xr[j] * inv * w[j];
  }
}

__global__ __launch_bounds__(256) void vec_add_kernel(float* __restrict__ a, const float* __restrict__ b, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] += b[i];
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ out, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

template <int FMT>
void launch_rows_t(const uint8_t* w, size_t row_bytes, int nb, const void* acts, size_t row_lo, size_t n_rows,
                   float* out, hipStream_t s) {
  const unsigned grid = (unsigned)((n_rows + kRowsPerWG - 1) / kRowsPerWG);
  hipLaunchKernelGGL((gemv_rows_kernel<FMT>), dim3(grid), dim3(64 * kRowsPerWG), 0, s, w, row_bytes, nb, acts,
                     (long)row_lo, (int)n_rows, out);
}


// ---- batched GEMV on int8 MFMA (gemv.rs:444-543, :616-651) ------------------
//
// out[i][a] = row(row_lo + i) . act_row(a) for a tile of 32 weight rows x
// 32 * W activation rows (one 32-row tile per wave) per workgroup. Every output is the
// scalar dot's f32 value bit for bit: the integer sums are exact (int8
// products, int32 accumulation) and the per-block float expression and the
// block order are the scalar kernel's.
//
// The k-quant integer sums go through v_mfma_i32_32x32x32_i8 with the
// sub-block scales folded into the weights (the A operand, weight rows =
// the MFMA's rows; the activations' int8 values are B, one column per
// activation row). sc * q does not fit in int8; the scale is split instead,
// so that each plane is a packed product with no carries between bytes:
//   Q4_K: sc = 8 sh + sl (sh, sl <= 7), q <= 15: planes sh*q, sl*q (<= 105)
//     and the mins m broadcast over their sub-block: sumi = 8 H + L,
//     sumi_mins = M (the Q8_K bsums are exactly the sub-block sums of the
//     activation values);
//   Q5_K: the same on q - 16 (sh*(q-16) in [-112, 105]) plus the scales
//     broadcast: sumi = 8 H + L + 16 S, sumi_mins = M;
//   Q6_K: sum_s sc_s (sum q a - 32 bsum_s) (dot.rs:150-179) is exactly
//     sum sc (q - 32) a; sc (q - 32) = 64 hi + lo (lo < 64): sumi = 64 H + L;
//   Q8_0: the weight bytes themselves, one MFMA per 32-weight block.
// The planes of one block (eight Q8_0 blocks) of the workgroup's 32 rows
// are built once in LDS, one thread per (row, 32-weight sub-block), and
// used by every activation tile of the workgroup.
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kBRows = 32;
constexpr int kPlaneRow = 272;  // 256 bytes + 16: 16-byte LDS reads of 32 rows spread over the banks

struct BatchedArgs {
  const uint8_t* w;
  size_t row_bytes;
  int nb;            // weight blocks per row (k-quant: 256 weights, Q8_0: 32)
  const void* acts;  // n_acts rows of nb Q8_K (k-quants) or Q8_0 blocks
  int n_acts;
  long row_lo;
  int n_rows;
  float* out;
  long ldo;
  int transposed;    // 0: out[i * ldo + a] (the reference's layout); 1: out[a * ldo + i]
  int accumulate;    // out += dot (one f32 add, as the prefill's residual add)
};

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

// 32 bytes at a 2-byte-aligned address as raw dwords (aligned-down reads
// plus a 2-byte tail, as load32_a2), with the realignment left to
// fix32_a2, so the loads can be issued one step ahead of their use.
struct Raw32 {
  uint32_t e[8];
  uint32_t tail;
  bool odd;
};
__device__ __forceinline__ Raw32 raw32_a2(const uint8_t* a) {
  Raw32 r;
  r.odd = ((uintptr_t)a & 2) != 0;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(a - (r.odd ? 2 : 0));
#pragma unroll
  for (int k = 0; k < 8; ++k) r.e[k] = p[k];
  r.tail = r.odd ? *reinterpret_cast<const uint16_t*>(a + 30) : 0u;
  return r;
}
__device__ __forceinline__ void fix32_a2(const Raw32& r, uint32_t (&w)[8]) {
#pragma unroll
  for (int k = 0; k < 7; ++k) w[k] = r.odd ? __builtin_amdgcn_alignbyte(r.e[k + 1], r.e[k], 2) : r.e[k];
  w[7] = r.odd ? (r.e[7] >> 16) | (r.tail << 16) : r.e[7];
}

// The bytes thread (r, j) needs to build its row's sub-block j of one block
// (or block j of a group of eight Q8_0 blocks), loaded one step ahead.
template <int FMT>
struct WRaw {
  uint32_t hdr[4];  // k-quants: d/dmin dword and the 12 scale bytes; Q6_K: scale pair, d
  uint32_t q[8];    // Q4_K/Q5_K quants
  uint32_t h[8];    // Q5_K high bits
  Raw32 a, b;       // Q6_K ql / qh; Q8_0 qs (a) and d (hdr[0])
};

template <int FMT>
__device__ __forceinline__ void load_wraw(const uint8_t* __restrict__ blk, int j, WRaw<FMT>& w) {
  if constexpr (FMT == RV_QF_Q4_K || FMT == RV_QF_Q5_K) {
    constexpr bool kQ5 = FMT == RV_QF_Q5_K;
    const uint32_t* hp = reinterpret_cast<const uint32_t*>(blk);
    w.hdr[0] = hp[0], w.hdr[1] = hp[1], w.hdr[2] = hp[2], w.hdr[3] = hp[3];
    const u32x4a* qp = reinterpret_cast<const u32x4a*>(blk + (kQ5 ? 48 : 16) + 32 * (j >> 1));
    const u32x4a q0 = qp[0], q1 = qp[1];
    w.q[0] = q0[0], w.q[1] = q0[1], w.q[2] = q0[2], w.q[3] = q0[3];
    w.q[4] = q1[0], w.q[5] = q1[1], w.q[6] = q1[2], w.q[7] = q1[3];
    if constexpr (kQ5) {
      const u32x4a* qh = reinterpret_cast<const u32x4a*>(blk + 16);
      const u32x4a h0 = qh[0], h1 = qh[1];
      w.h[0] = h0[0], w.h[1] = h0[1], w.h[2] = h0[2], w.h[3] = h0[3];
      w.h[4] = h1[0], w.h[5] = h1[1], w.h[6] = h1[2], w.h[7] = h1[3];
    }
  } else if constexpr (FMT == RV_QF_Q6_K) {
    const int half = j >> 2, grp = j & 3;
    w.a = raw32_a2(blk + 64 * half + 32 * (grp & 1));
    w.b = raw32_a2(blk + 128 + 32 * half);
    w.hdr[0] = *reinterpret_cast<const uint16_t*>(blk + 192 + 2 * j);
    w.hdr[1] = *reinterpret_cast<const uint16_t*>(blk + 208);
  } else {
    w.a = raw32_a2(blk + 2);
    w.hdr[0] = *reinterpret_cast<const uint16_t*>(blk);
  }
}

// Thread (r, j) writes the 32 plane bytes of its row's sub-block j
// (weights 32j .. 32j+31 of the block) and, for j == 0, the row's block
// scalars (Q8_0: block j's d).
template <int FMT>
__device__ __forceinline__ void build_planes(const WRaw<FMT>& wr, int j, int8_t (*pl)[kBRows][kPlaneRow], int r,
                                             float (*sd)[kBRows]) {
  uint32_t q[8];
  int sc[2], m = 0;
  if constexpr (FMT == RV_QF_Q4_K || FMT == RV_QF_Q5_K) {
    const uint32_t s3[3] = {wr.hdr[1], wr.hdr[2], wr.hdr[3]};
    scale_min_k4(j, s3, sc[0], m);
    sc[1] = sc[0];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      q[k] = (j & 1) ? (wr.q[k] >> 4) & 0x0F0F0F0Fu : wr.q[k] & 0x0F0F0F0Fu;
      if constexpr (FMT == RV_QF_Q5_K) q[k] |= ((wr.h[k] >> j) & 0x01010101u) << 4;
    }
    if (j == 0) {
      sd[0][r] = f16_bits_to_f32(wr.hdr[0]);
      sd[1][r] = f16_bits_to_f32(wr.hdr[0] >> 16);
    }
  } else if constexpr (FMT == RV_QF_Q6_K) {
    const int grp = j & 3;
    uint32_t ql[8], qh[8];
    fix32_a2(wr.a, ql);
    fix32_a2(wr.b, qh);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t nib = (grp >> 1) ? (ql[k] >> 4) & 0x0F0F0F0Fu : ql[k] & 0x0F0F0F0Fu;
      q[k] = nib | (((qh[k] >> (2 * grp)) & 0x03030303u) << 4);
    }
    sc[0] = (int)(int8_t)(wr.hdr[0] & 0xFF);
    sc[1] = (int)(int8_t)(wr.hdr[0] >> 8);
    if (j == 0) sd[0][r] = f16_bits_to_f32(wr.hdr[1]);
  } else {
    fix32_a2(wr.a, q);
    sd[j][r] = f16_bits_to_f32(wr.hdr[0]);
  }
  auto plane = [&](int p) { return reinterpret_cast<u32x4a*>(&pl[p][r][32 * j]); };
  auto put = [&](int p, const uint32_t (&v)[8]) {
    plane(p)[0] = u32x4a{v[0], v[1], v[2], v[3]};
    plane(p)[1] = u32x4a{v[4], v[5], v[6], v[7]};
  };
  if constexpr (FMT == RV_QF_Q8_0) {
    put(0, q);
  } else if constexpr (FMT == RV_QF_Q4_K || FMT == RV_QF_Q5_K) {
    // q bytes times a 3-bit scale part: four exact byte products per dword.
    const uint32_t sh = (uint32_t)sc[0] >> 3, sl = (uint32_t)sc[0] & 7;
    uint32_t h[8], l[8], mm[8], ss[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (FMT == RV_QF_Q4_K) {
        h[k] = q[k] * sh;
        l[k] = q[k] * sl;
      } else {
        // bytes s*q + (128 - 16 s) in [16, 233] (no carries), then the top
        // bit flipped: the signed bytes s*(q - 16).
        h[k] = (q[k] * sh + (128u - 16u * sh) * 0x01010101u) ^ 0x80808080u;
        l[k] = (q[k] * sl + (128u - 16u * sl) * 0x01010101u) ^ 0x80808080u;
        ss[k] = (uint32_t)sc[0] * 0x01010101u;
      }
      mm[k] = (uint32_t)m * 0x01010101u;
    }
    put(0, h);
    put(1, l);
    put(2, mm);
    if constexpr (FMT == RV_QF_Q5_K) put(3, ss);
  } else {
    uint32_t h[8], l[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int s2 = sc[k >> 2];  // the first 16 weights take sc[0], the rest sc[1]
      int hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = s2 * ((int)((q[k] >> (8 * e)) & 0xFF) - 32);
        hi[e] = v >> 6;  // arithmetic shift: floor, so lo = v - 64 hi is in [0, 64)
        lo[e] = v & 63;
      }
      h[k] = pack4(hi[0], hi[1], hi[2], hi[3]);
      l[k] = pack4(lo[0], lo[1], lo[2], lo[3]);
    }
    put(0, h);
    put(1, l);
  }
}

// The activation operands of one step for one tile: lane (li, kh) holds
// activation row li's bytes 16 kh .. 16 kh + 15 of each 32-value chunk.
template <bool Q80>
__device__ __forceinline__ void load_acts(const void* __restrict__ acts, int act, int nb, int step, i32x4 (&bq)[8],
                                          float (&da)[8], int kh) {
  if constexpr (Q80) {
    const rv_block_q8_0* y = reinterpret_cast<const rv_block_q8_0*>(acts) + (size_t)act * nb;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const rv_block_q8_0* yb = y + min(8 * step + c, nb - 1);
      const u32x4a v = *reinterpret_cast<const u32x4a*>(yb->qs + 16 * kh);
      bq[c] = i32x4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
      da[c] = yb->d;
    }
  } else {
    const rv_block_q8_k* y = reinterpret_cast<const rv_block_q8_k*>(acts) + (size_t)act * nb + step;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u32x4a v = *reinterpret_cast<const u32x4a*>(y->qs + 32 * c + 16 * kh);
      bq[c] = i32x4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
    }
    da[0] = y->d;
  }
}

template <int FMT, int W>
__global__ __launch_bounds__(64 * W) void gemv_batched_kernel(BatchedArgs a) {
#pragma clang fp contract(off)
  constexpr bool kQ80 = FMT == RV_QF_Q8_0;
  constexpr int kPlanes = kQ80 ? 1 : FMT == RV_QF_Q6_K ? 2 : FMT == RV_QF_Q5_K ? 4 : 3;
  constexpr int BB = FMT == RV_QF_Q4_K ? 144 : FMT == RV_QF_Q5_K ? 176 : FMT == RV_QF_Q6_K ? 210 : 34;
  constexpr int NB = 4 / W;  // (row, sub-block) build tasks per thread: 256 per step
  __shared__ __attribute__((aligned(16))) int8_t pl[kPlanes][kBRows][kPlaneRow];
  // Per-row block scalars, row-minor so a lane's four consecutive output
  // rows come in one 16-byte read: k-quants [0] d and [1] dmin; Q8_0 [c]
  // the d of block c of the group.
  __shared__ __attribute__((aligned(16))) float sd[8][kBRows];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, kh = lane >> 5;
  const int row0 = blockIdx.x * kBRows;
  // Builder role: task u = tid + 64 W n -> (row u >> 3, sub-block u & 7);
  // rows past the range re-read the last row (their outputs are not stored).
  const uint8_t* wrow[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n)
    wrow[n] = a.w + (size_t)(a.row_lo + min(row0 + ((tid + 64 * W * n) >> 3), a.n_rows - 1)) * a.row_bytes;
  const int bj = tid & 7;  // the same for every task of the thread (64 W is a multiple of 8)
  auto wblk = [&](int n, int step) {
    return kQ80 ? wrow[n] + (size_t)min(8 * step + bj, a.nb - 1) * BB : wrow[n] + (size_t)step * BB;
  };
  const int act = min((int)blockIdx.y * 32 * W + 32 * wave + li, a.n_acts - 1);
  float sumf[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sumf[r] = 0.f;
  const int n_steps = kQ80 ? (a.nb + 7) / 8 : a.nb;
  // Software pipeline: the weight bytes of steps + 1 .. + 2 and the
  // activation operands of step + 1 are in flight while step's planes are
  // built and its MFMAs run (a weight block's memory round trip is longer
  // than one step). The register rings are indexed by the unrolled u. Every
  // load is issued unconditionally (steps past the end re-read the last
  // one): a conditional load would make the compiler merge the old and new
  // registers after the branch and wait for the load right there.
  constexpr int DW = 3, DA = 2;
  const int last = n_steps - 1;
  WRaw<FMT> wr[DW][NB];
#pragma unroll
  for (int u = 0; u < DW; ++u)
#pragma unroll
    for (int n = 0; n < NB; ++n) load_wraw<FMT>(wblk(n, min(u, last)), bj, wr[u][n]);
  i32x4 bq[DA][8];
  float da[DA][8];
#pragma unroll
  for (int u = 0; u < DA; ++u) load_acts<kQ80>(a.acts, act, a.nb, min(u, last), bq[u], da[u], kh);
  for (int s0 = 0; s0 < n_steps; s0 += DW * DA) {
#pragma unroll
  for (int u = 0; u < DW * DA; ++u) {
    const int step = s0 + u;
    if (step >= n_steps) break;
    const int uw = u % DW, ua = u % DA;
#pragma unroll
    for (int n = 0; n < NB; ++n) build_planes<FMT>(wr[uw][n], bj, pl, (tid + 64 * W * n) >> 3, sd);
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NB; ++n) load_wraw<FMT>(wblk(n, min(step + DW, last)), bj, wr[uw][n]);
    i32x4 cur[8];
    float dcur[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) cur[c] = bq[ua][c], dcur[c] = da[ua][c];
    load_acts<kQ80>(a.acts, act, a.nb, min(step + DA, last), bq[ua], da[ua], kh);
    // Lane (li, kh) owns output rows 8 g + 4 kh + e (e < 4) of the tile, g < 4.
    auto rows4 = [&](int k, int g) { return *reinterpret_cast<const f32x4*>(&sd[k][8 * g + 4 * kh]); };
    auto aop = [&](int p, int c) { return *reinterpret_cast<const i32x4*>(&pl[p][li][32 * c + 16 * kh]); };
    if constexpr (kQ80) {
      const int nblk = min(8, a.nb - 8 * step);
      i32x4 wa = aop(0, 0);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        i32x16 acc = {};
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa, cur[c], acc, 0, 0, 0);
        if (c + 1 < 8) wa = aop(0, c + 1);  // in flight under this MFMA
        f32x4 dw[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) dw[g] = rows4(c, g);
        if (c < nblk) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sumf[r] += (float)acc[r] * (dw[r >> 2][r & 3] * dcur[c]);
        }
      }
    } else {
      f32x4 dw[4], dm[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        dw[g] = rows4(0, g);
        if constexpr (FMT != RV_QF_Q6_K) dm[g] = rows4(1, g);
      }
      i32x16 acc[kPlanes];
#pragma unroll
      for (int p = 0; p < kPlanes; ++p) acc[p] = i32x16{};
      i32x4 wa[kPlanes], wn[kPlanes];
#pragma unroll
      for (int p = 0; p < kPlanes; ++p) wa[p] = aop(p, 0);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if (c + 1 < 8) {
#pragma unroll
          for (int p = 0; p < kPlanes; ++p) wn[p] = aop(p, c + 1);  // in flight under chunk c's MFMAs
        }
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) acc[p] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa[p], cur[c], acc[p], 0, 0, 0);
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) wa[p] = wn[p];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float dr = dw[r >> 2][r & 3];
        if constexpr (FMT == RV_QF_Q6_K) {
          const int sumi = 64 * acc[0][r] + acc[1][r];
          sumf[r] += dr * dcur[0] * (float)sumi;
        } else {
          int sumi = 8 * acc[0][r] + acc[1][r];
          if constexpr (FMT == RV_QF_Q5_K) sumi += 16 * acc[3][r];
          const float d = dr * dcur[0], dmin = dm[r >> 2][r & 3] * dcur[0];
          sumf[r] += d * (float)sumi - dmin * (float)acc[2][r];
        }
      }
    }
    __syncthreads();  // the next step's planes overwrite these
  }
  }
  const int act_out = (int)blockIdx.y * 32 * W + 32 * wave + li;
  if (act_out >= a.n_acts) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = row0 + 8 * (r >> 2) + 4 * kh + (r & 3);
    if (i < a.n_rows) {
      float* o = a.out + (a.transposed ? (size_t)act_out * a.ldo + i : (size_t)i * a.ldo + act_out);
      *o = a.accumulate ? *o + sumf[r] : sumf[r];
    }
  }
}
}  // namespace

HipStatus launch_quantize_q8_k(const float* x, rv_block_q8_k* out, size_t n_blocks, hipStream_t s) {
  HipStatus st;
  if (n_blocks == 0) return st;
  hipLaunchKernelGGL(quantize_q8_k_kernel, dim3((unsigned)((n_blocks + 3) / 4)), dim3(256), 0, s, x, out,
                     (int)n_blocks);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "quantize_q8_k launch";
  return st;
}

HipStatus launch_quantize_q8_0(const float* x, rv_block_q8_0* out, size_t n_blocks, hipStream_t s) {
  HipStatus st;
  if (n_blocks == 0) return st;
  hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((n_blocks * 32 + 255) / 256)), dim3(256), 0, s, x, out,
                     (int)n_blocks);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "quantize_q8_0 launch";
  return st;
}

HipStatus launch_gemv_rows(uint32_t fmt, const uint8_t* w, size_t row_bytes, size_t in_dim, const void* acts,
                           size_t row_lo, size_t n_rows, float* out, hipStream_t s) {
  HipStatus st;
  if (n_rows == 0 || in_dim == 0) return st;
  const int nb = (int)(in_dim / (fmt == RV_QF_Q8_0 ? 32 : 256));
  switch (fmt) {
    case RV_QF_Q4_K: launch_rows_t<RV_QF_Q4_K>(w, row_bytes, nb, acts, row_lo, n_rows, out, s); break;
    case RV_QF_Q5_K: launch_rows_t<RV_QF_Q5_K>(w, row_bytes, nb, acts, row_lo, n_rows, out, s); break;
    case RV_QF_Q6_K: launch_rows_t<RV_QF_Q6_K>(w, row_bytes, nb, acts, row_lo, n_rows, out, s); break;
    default: launch_rows_t<RV_QF_Q8_0>(w, row_bytes, nb, acts, row_lo, n_rows, out, s);
  }
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "gemv launch";
  return st;
}

HipStatus launch_fill_zero(float* out, size_t n, hipStream_t s) {
  HipStatus st;
  if (n == 0) return st;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, (long)n);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "fill launch";
  return st;
}

HipStatus launch_fused_proj(const FusedProjArgs& a, hipStream_t s) {
  HipStatus st;
  long rows = 0;
  for (int i = 0; i < a.n_seg; ++i) rows += a.n_rows[i];
  if (rows == 0) return st;
  const dim3 grid((unsigned)((rows + kFusedWaves - 1) / kFusedWaves));
  if (a.norm_w)
    hipLaunchKernelGGL(fused_proj_kernel<true>, grid, dim3(64 * kFusedWaves), 0, s, a);
  else
    hipLaunchKernelGGL(fused_proj_kernel<false>, grid, dim3(64 * kFusedWaves), 0, s, a);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "fused projection launch";
  return st;
}

HipStatus launch_rmsnorm(const float* x, const float* w, float eps, size_t n, float* out, hipStream_t s) {
  HipStatus st;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, x, w, eps, (int)n, out);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "rmsnorm launch";
  return st;
}

HipStatus launch_vec_add(float* a, const float* b, size_t n, hipStream_t s) {
  HipStatus st;
  if (n == 0) return st;
  hipLaunchKernelGGL(vec_add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, (long)n);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "vec_add launch";
  return st;
}

template <int FMT, int W>
void launch_batched_t(const BatchedArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.n_rows + kBRows - 1) / kBRows), (unsigned)((a.n_acts + 32 * W - 1) / (32 * W)));
  hipLaunchKernelGGL((gemv_batched_kernel<FMT, W>), grid, dim3(64 * W), 0, s, a);
}

template <int FMT>
void launch_batched_f(const BatchedArgs& a, hipStream_t s) {
  // Four 32-activation tiles per workgroup share its planes; Q8_0 matrices
  // with few row tiles (the k projection: 16) take one tile per workgroup
  // instead, four times the workgroups (its plane build is a copy).
  const long row_tiles = (a.n_rows + kBRows - 1) / kBRows;
  if (FMT == RV_QF_Q8_0 && row_tiles * ((a.n_acts + 127) / 128) < 256)
    launch_batched_t<FMT, 1>(a, s);
  else
    launch_batched_t<FMT, 4>(a, s);
}

HipStatus launch_gemv_batched(uint32_t fmt, const uint8_t* w, size_t row_bytes, size_t in_dim, const void* acts,
                              size_t n_acts, size_t row_lo, size_t n_rows, float* out, size_t ldo, bool transposed,
                              hipStream_t s, bool accumulate) {
  HipStatus st;
  if (n_rows == 0 || n_acts == 0) return st;
  BatchedArgs a{w, row_bytes, (int)(in_dim / (fmt == RV_QF_Q8_0 ? 32 : 256)), acts, (int)n_acts, (long)row_lo,
                (int)n_rows, out, (long)ldo, transposed ? 1 : 0, accumulate ? 1 : 0};
  switch (fmt) {
    case RV_QF_Q4_K: launch_batched_f<RV_QF_Q4_K>(a, s); break;
    case RV_QF_Q5_K: launch_batched_f<RV_QF_Q5_K>(a, s); break;
    case RV_QF_Q6_K: launch_batched_f<RV_QF_Q6_K>(a, s); break;
    default: launch_batched_f<RV_QF_Q8_0>(a, s);
  }
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "batched gemv launch";
  return st;
}

HipStatus launch_rmsnorm_rows(const float* x, const float* w, float eps, size_t n_rows, size_t n, float* out,
                              hipStream_t s) {
  HipStatus st;
  if (n_rows == 0) return st;
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)n_rows), dim3(256), 0, s, x, w, eps, (int)n, out);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "rmsnorm rows launch";
  return st;
}

HipStatus launch_quantize_both(const float* x, rv_block_q8_k* ok, rv_block_q8_0* o0, size_t n_k_blocks,
                               hipStream_t s) {
  HipStatus st;
  if (n_k_blocks == 0) return st;
  hipLaunchKernelGGL(quantize_both_kernel, dim3((unsigned)((n_k_blocks + 3) / 4)), dim3(256), 0, s, x, ok, o0,
                     (int)n_k_blocks);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "quantize launch";
  return st;
}

}  // namespace rv

