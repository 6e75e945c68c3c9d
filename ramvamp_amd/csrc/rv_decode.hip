// rv_decode.hip — single-token GQA decode attention on gfx950.
//
// Replaces attention_body / qk_scores / softmax / v_reduce
// (crates/core/src/kernels/attention.rs:1075-1303) for the decode and
// position-limited forms.
//
// Fast path (head_dim 128, any group): one workgroup of W waves per (kv
// head, subgroup of G query heads, split of the position axis). A K or V
// row's 128-element head slice is read by one 16-lane group, 8 elements (16
// or 32 bytes) per lane, and serves the subgroup's G heads from registers.
// QK dots reduce over the 16 lanes with DPP; softmax is online (running max
// and sum per query head, exp2 with log2(e) folded into q). The 4*W row
// groups of a workgroup merge through LDS; the splits of one (kv head,
// subgroup) are merged by a second kernel with an fp32 log-sum-exp combine
// (the kernel boundary makes the partials visible: an in-kernel hand-off
// would need agent-scope fences, which write back and invalidate the L2 and
// cost more than the second launch).
//
// Why subgroups: one CU streams only ~10-25 GB/s, so the merge must read
// little (splits x G x 520 bytes) while the grid stays wide enough to put
// every CU on the K/V stream. Subgroups of one (kv head, split) read the same
// rows; the grid places them on one XCD so its L2 serves the repeats and HBM
// sees each K/V byte once.
//
// Generic path (any head_dim, any group): scores, softmax and the V
// reduction as three kernels in the reference's own order — f32 dots with
// i ascending and separate multiply/add, an f64 exp/sum softmax, and the V
// sum over t ascending per output element.
#include "rv_device.hpp"
#include "rv_internal.hpp"

#include <algorithm>

namespace rv {
namespace {

constexpr int kD = 128;                     // head_dim of the fast path
constexpr int kLPR = 16;                    // lanes per K/V row (8 elements each)
constexpr int kMaxSplits = 256;             // splits per kv head the merge stages in LDS
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegSentinel = -1.0e30f;    // finite "no position yet" max

// Partial layout per (kv head, split): o[G][kD] then (m, l)[G], padded to a
// 16-byte multiple so every partial row starts 16-byte aligned.
__host__ __device__ constexpr int part_stride_of(int g) { return g * kD + (2 * g + 3) / 4 * 4; }
template <int G>
constexpr int part_stride() {
  return part_stride_of(G);
}

// Element e (0..7) of the 8 a lane holds of a row's 128-element head slice:
// f32 rows as two 16-byte pieces 256 bytes apart (each load instruction then
// reads 256 contiguous bytes of every row), f16 rows as one 16-byte piece.
template <typename T>
__device__ __forceinline__ int lane_d(int c, int e);
template <>
__device__ __forceinline__ int lane_d<float>(int c, int e) {
  return e < 4 ? 4 * c + e : 64 + 4 * c + (e - 4);
}
template <>
__device__ __forceinline__ int lane_d<_Float16>(int c, int e) {
  return 8 * c + e;
}
template <typename T>
__device__ __forceinline__ void load_row8(const T* __restrict__ row, int c, float (&x)[8]);
template <>
__device__ __forceinline__ void load_row8<float>(const float* __restrict__ row, int c, float (&x)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(row + 4 * c);
  const f32x4 b = *reinterpret_cast<const f32x4*>(row + 64 + 4 * c);
  x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
  x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
}
template <>
__device__ __forceinline__ void load_row8<_Float16>(const _Float16* __restrict__ row, int c, float (&x)[8]) {
  const f16x8 h = *reinterpret_cast<const f16x8*>(row + 8 * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)h[i];
}

// One workgroup per (kv head, subgroup of G query heads, split). The 1-D
// grid puts the n_hg subgroups of one (kv head, split) unit on the same XCD
// (workgroups are dispatched round-robin over the 8 XCDs, so equal block ids
// mod 8 share an L2) and in the same dispatch round: the subgroups read the
// same K/V rows, and L2 serves all but the first. With one split the
// workgroup writes `out`; otherwise its partial (o, max, sum) row, merged by
// decode_merge_kernel.
template <typename T, int G, int R, int W>
__global__ __launch_bounds__(W * 64) void decode_split_kernel(const float* __restrict__ q,
                                                              const T* __restrict__ kl,
                                                              const T* __restrict__ vl, int kv_dim,
                                                              int positions, int split_len,
                                                              int n_splits, int n_units, int group,
                                                              int n_hg, int kv_lo, float qscale,
                                                              float* __restrict__ part,
                                                              float* __restrict__ out) {
  constexpr int NT = W * 64;
  constexpr int kRowsPerStep = W * (64 / kLPR);
  constexpr int NO = G * kD / 4;  // float4 outputs per subgroup
  const int b = blockIdx.x;
  const int hg = (b % (8 * n_hg)) / 8;
  const int u = (b / (8 * n_hg)) * 8 + b % 8;
  if (u >= n_units) return;
  const int split = u % n_splits;
  const int hidx = u / n_splits;  // kv head within the range
  const int kvh = kv_lo + hidx;
  const int job = hidx * n_hg + hg;          // (kv head, subgroup)
  const int h0 = hidx * group + hg * G;      // first q head of the subgroup, within the range
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & (kLPR - 1);
  const int row = wave * (64 / kLPR) + (lane >> 4);
  const int t_begin = split * split_len;
  const int t_end = min(positions, t_begin + split_len);

  float qr[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qp = q + (size_t)(kv_lo * group + h0 + g) * kD;
#pragma unroll
    for (int e = 0; e < 8; ++e) qr[g][e] = qp[lane_d<T>(c, e)] * qscale;
  }
  float o[G][8], m[G], l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegSentinel;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }

  const size_t col = (size_t)kvh * kD;
  constexpr int kBlock = R * kRowsPerStep;  // rows per block
  // Rows past the split re-read its last row (in bounds, branch-free); their
  // scores are masked in compute_block.
  auto load_block = [&](int t0, float (&kx)[R][8], float (&vx)[R][8]) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int t = min(t0 + j * kRowsPerStep + row, t_end - 1);
      load_row8<T>(kl + (size_t)t * kv_dim + col, c, kx[j]);
      load_row8<T>(vl + (size_t)t * kv_dim + col, c, vx[j]);
    }
  };
  auto compute_block = [&](int t0, const float (&kx)[R][8], const float (&vx)[R][8]) {
    float s[R][G];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const bool valid = t0 + j * kRowsPerStep + row < t_end;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += qr[g][e] * kx[j][e];
        acc = group_sum<kLPR>(acc);
        s[j][g] = valid ? acc : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mb = s[0][g];
#pragma unroll
      for (int j = 1; j < R; ++j) mb = fmaxf(mb, s[j][g]);
      const float mn = fmaxf(m[g], mb);
      const float a = exp2f(m[g] - mn);
      l[g] *= a;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= a;
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const float p = exp2f(s[j][g] - mn);
        l[g] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] += p * vx[j][e];
      }
      m[g] = mn;
    }
  };
  // Software pipeline: the next block's loads are in flight while the
  // current block is computed (ping-pong register buffers A and B).
  float ka[R][8], va[R][8], kb[R][8], vb[R][8];
  load_block(t_begin, ka, va);
  for (int t0 = t_begin; t0 < t_end; t0 += 2 * kBlock) {
    const bool has_b = t0 + kBlock < t_end;
    if (has_b) load_block(t0 + kBlock, kb, vb);
    compute_block(t0, ka, va);
    if (!has_b) break;
    if (t0 + 2 * kBlock < t_end) load_block(t0 + 2 * kBlock, ka, va);
    compute_block(t0 + kBlock, kb, vb);
  }

  // Merge the four row groups of this wave (lanes 16 and 32 apart).
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off, 64);
      const float lo = __shfl_xor(l[g], off, 64);
      const float mn = fmaxf(m[g], mo);
      const float a = exp2f(m[g] - mn), bb = exp2f(mo - mn);
      l[g] = l[g] * a + lo * bb;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] = o[g][e] * a + __shfl_xor(o[g][e], off, 64) * bb;
      m[g] = mn;
    }
  }

  __shared__ __attribute__((aligned(16))) float sm_o[W][G][kD];
  __shared__ float sm_ml[W][G][2];
  if (lane < kLPR) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_o[wave][g][lane_d<T>(c, e)] = o[g][e];
      if (c == 0) {
        sm_ml[wave][g][0] = m[g];
        sm_ml[wave][g][1] = l[g];
      }
    }
  }
  __syncthreads();

  // Merge the W waves: thread -> (head g, 4 consecutive d).
  float* mine = part + ((size_t)job * n_splits + split) * part_stride<G>();
  for (int j = tid; j < NO; j += NT) {
    const int g = j / (kD / 4), d = (j % (kD / 4)) * 4;
    float M = sm_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < W; ++w) M = fmaxf(M, sm_ml[w][g][0]);
    float L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float a = exp2f(sm_ml[w][g][0] - M);
      L += sm_ml[w][g][1] * a;
      O += *reinterpret_cast<const f32x4*>(&sm_o[w][g][d]) * a;
    }
    if (n_splits == 1) {
      const f32x4 r = O / L;  // out may be only 4-byte aligned
      float* op = &out[(size_t)(h0 + g) * kD + d];
      op[0] = r[0];
      op[1] = r[1];
      op[2] = r[2];
      op[3] = r[3];
    } else {
      *reinterpret_cast<f32x4*>(&mine[g * kD + d]) = O;
      if (d == 0) {
        mine[G * kD + 2 * g] = M;
        mine[G * kD + 2 * g + 1] = L;
      }
    }
  }
}

// ---- MFMA path ------------------------------------------------------------------

// 32 consecutive plane elements widened to f32.
template <typename T>
__device__ __forceinline__ void load32(const T* __restrict__ p, float (&x)[32]);
template <>
__device__ __forceinline__ void load32<float>(const float* __restrict__ p, float (&x)[32]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f32x4 a = reinterpret_cast<const f32x4*>(p)[i];
    x[4 * i] = a[0];
    x[4 * i + 1] = a[1];
    x[4 * i + 2] = a[2];
    x[4 * i + 3] = a[3];
  }
}
template <>
__device__ __forceinline__ void load32<_Float16>(const _Float16* __restrict__ p, float (&x)[32]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x8 a = reinterpret_cast<const f16x8*>(p)[i];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[8 * i + j] = (float)a[j];
  }
}

// LDS row stride of a staged 16 x 128 tile, in floats: 4 words of padding
// put the 16 rows read at one column into 16 different bank groups.
constexpr int kTileStride = kD + 4;

// One 16-position K or V tile (16 rows x 128 elements of one kv head) in
// staging registers, loaded with whole rows per instruction: f32 lane i of
// step j holds row 2j + i/32, columns 4*(i%32)..+3; f16 lane i of step j
// holds row 4j + i/16, columns 8*(i%16)..+7.
template <typename T>
struct TileRegs;
template <>
struct TileRegs<float> {
  static constexpr int kSteps = 8;
  f32x4 r[8];
  __device__ void load(const float* __restrict__ plane, int kv_dim, size_t col, int t0, int t_last, int lane) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = min(t0 + 2 * j + (lane >> 5), t_last);
      r[j] = *reinterpret_cast<const f32x4*>(plane + (size_t)row * kv_dim + col + 4 * (lane & 31));
    }
  }
  __device__ void store(float (*lds)[kTileStride], int lane) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<f32x4*>(&lds[2 * j + (lane >> 5)][4 * (lane & 31)]) = r[j];
  }
};
template <>
struct TileRegs<_Float16> {
  f16x8 r[4];
  __device__ void load(const _Float16* __restrict__ plane, int kv_dim, size_t col, int t0, int t_last, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = min(t0 + 4 * j + (lane >> 4), t_last);
      r[j] = *reinterpret_cast<const f16x8*>(plane + (size_t)row * kv_dim + col + 8 * (lane & 15));
    }
  }
  __device__ void store(float (*lds)[kTileStride], int lane) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 a, b;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = (float)r[j][e];
        b[e] = (float)r[j][4 + e];
      }
      float* dst = &lds[4 * j + (lane >> 4)][8 * (lane & 15)];
      *reinterpret_cast<f32x4*>(dst) = a;
      *reinterpret_cast<f32x4*>(dst + 4) = b;
    }
  }
};

// One workgroup of W waves per (kv head, split); all `group` (<= 16) query
// heads of the kv head are the 16 columns of fp32 MFMA tiles
// (v_mfma_f32_16x16x4_f32: exact fp32 products, fp32 accumulation). Wave w
// takes the split's 16-position tiles w, w+W, ...; each tile's K and V rows
// are read whole-row-per-instruction into registers (the next tile's loads
// are issued before the current tile is computed), converted to f32 and
// staged in the wave's own LDS region, from which the MFMA operands are read:
//   S^T[t][m] = sum_d K[t][d] Q[m][d]: 32 MFMAs; A slot (lane t + 16*kg,
//     step s) is K[t][32*kg + s], B is q (loaded once, log2(e)*scale folded);
//   online softmax on the accumulator: lane l holds rows 4*(l/16) + i of
//     column l % 16, so a column's max needs two cross-lane swaps and every
//     exp is computed once;
//   O^T[d][m] += sum_t V[t][d] P[m][t]: 8 x 4 MFMAs; the accumulator layout
//     of S^T is exactly the B layout P^T needs, so P never moves.
// The waves merge through LDS; the workgroup writes `out` (one split) or its
// partial (o, max, sum) row for decode_merge_kernel.
template <typename T, int W>
__global__ __launch_bounds__(W * 64) void decode_mfma_kernel(const float* __restrict__ q, const T* __restrict__ kl,
                                                             const T* __restrict__ vl, int kv_dim, int positions,
                                                             int split_len, int n_splits, int group, int kv_lo,
                                                             float qscale, float* __restrict__ part,
                                                             float* __restrict__ out) {
  constexpr int NT = W * 64;
  __shared__ __attribute__((aligned(16))) float sm_kv[W][2][16][kTileStride];
  __shared__ float sm_ml[W][16][2];
  const int split = blockIdx.x % n_splits;
  const int hidx = blockIdx.x / n_splits;  // kv head within the range
  const int kvh = kv_lo + hidx;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lm = lane & 15, kg = lane >> 4;
  const int t_begin = split * split_len;
  const int t_end = min(positions, t_begin + split_len);
  const bool col_ok = lm < group;
  const size_t col = (size_t)kvh * kD;

  float qb[32];
  {
    const float* qp = q + (size_t)(kvh * group + (col_ok ? lm : 0)) * kD + kg * 32;
#pragma unroll
    for (int s = 0; s < 32; ++s) qb[s] = col_ok ? qp[s] * qscale : 0.f;
  }
  f32x4 o[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) o[ds] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegSentinel, l_run = 0.f;

  float (*ks)[kTileStride] = sm_kv[wave][0];
  float (*vs)[kTileStride] = sm_kv[wave][1];
  TileRegs<T> kr, vr;
  int t0 = t_begin + wave * 16;
  if (t0 < t_end) {
    kr.load(kl, kv_dim, col, t0, t_end - 1, lane);
    vr.load(vl, kv_dim, col, t0, t_end - 1, lane);
  }
  for (; t0 < t_end; t0 += W * 16) {
    // The wave's LDS region is its own, and one wave's LDS accesses complete
    // in order, so no barrier is needed between the store and the reads.
    kr.store(ks, lane);
    vr.store(vs, lane);
    const int tn = t0 + W * 16;
    if (tn < t_end) {
      kr.load(kl, kv_dim, col, tn, t_end - 1, lane);
      vr.load(vl, kv_dim, col, tn, t_end - 1, lane);
    }
    float ka[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&ks[lm][kg * 32 + 4 * i]);
      ka[4 * i] = a[0];
      ka[4 * i + 1] = a[1];
      ka[4 * i + 2] = a[2];
      ka[4 * i + 3] = a[3];
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 32; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[s], qb[s], acc, 0, 0, 0);
    float x[4], mx = kNegSentinel;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = (t0 + kg * 4 + i < t_end) ? acc[i] : -INFINITY;
      mx = fmaxf(mx, x[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - mn);
    m_run = mn;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = exp2f(x[i] - mn);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
      o[ds] *= alpha;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        o[ds] = __builtin_amdgcn_mfma_f32_16x16x4f32(vs[kg * 4 + s][ds * 16 + lm], p[s], o[ds], 0, 0, 0);
    }
  }
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // Merge the W waves through LDS (the tile regions are reused).
  __syncthreads();
  float (*so)[kTileStride] = sm_kv[wave][0];  // [16 heads][128 d]
  if (col_ok) {
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
#pragma unroll
      for (int i = 0; i < 4; ++i) so[lm][ds * 16 + kg * 4 + i] = o[ds][i];
    if (kg == 0) {
      sm_ml[wave][lm][0] = m_run;
      sm_ml[wave][lm][1] = l_run;
    }
  }
  __syncthreads();
  const int stride = part_stride_of(group);
  float* mine = part + ((size_t)hidx * n_splits + split) * stride;
  for (int j = tid; j < group * (kD / 4); j += NT) {
    const int g = j / (kD / 4), d = (j % (kD / 4)) * 4;
    float M = sm_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < W; ++w) M = fmaxf(M, sm_ml[w][g][0]);
    float L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float a = exp2f(sm_ml[w][g][0] - M);
      L += sm_ml[w][g][1] * a;
      O += *reinterpret_cast<const f32x4*>(&sm_kv[w][0][g][d]) * a;
    }
    if (n_splits == 1) {
      const f32x4 r = O / L;  // out may be only 4-byte aligned
      float* op = &out[(size_t)(hidx * group + g) * kD + d];
      op[0] = r[0];
      op[1] = r[1];
      op[2] = r[2];
      op[3] = r[3];
    } else {
      *reinterpret_cast<f32x4*>(&mine[g * kD + d]) = O;
      if (d == 0) {
        mine[group * kD + 2 * g] = M;
        mine[group * kD + 2 * g + 1] = L;
      }
    }
  }
}

// fp32 log-sum-exp merge of the splits of every (kv head, subgroup of G
// heads): one 256-thread workgroup per (subgroup, head, 64-column half). The
// four waves take every fourth split and fold them online; their loads do
// not depend on one another, so one round trip brings them all. The waves
// then merge through LDS.
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part, int n_splits, int stride,
                                                           int G, int group, int n_hg, float* __restrict__ out) {
  const int b = blockIdx.x;
  const int half = b & 1, jg = b >> 1;
  const int g = jg % G, job = jg / G;
  const int hidx = job / n_hg, hg = job % n_hg;
  const int h = hidx * group + hg * G + g;  // q head within the range
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int d = half * 64 + lane;
  const float* base = part + (size_t)job * n_splits * stride;
  float M = kNegSentinel, L = 0.f, O = 0.f;
#pragma unroll 16
  for (int sp = wave; sp < n_splits; sp += 4) {
    const float* ps = base + (size_t)sp * stride;
    const float m = ps[G * kD + 2 * g], l = ps[G * kD + 2 * g + 1], o = ps[g * kD + d];
    const float mn = fmaxf(M, m);
    const float a = exp2f(M - mn), c = exp2f(m - mn);
    L = L * a + l * c;
    O = O * a + o * c;
    M = mn;
  }
  __shared__ float sm[3][4][64];
  sm[0][wave][lane] = M;
  sm[1][wave][lane] = L;
  sm[2][wave][lane] = O;
  __syncthreads();
  if (wave == 0) {
    float Mt = sm[0][0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) Mt = fmaxf(Mt, sm[0][w][lane]);
    float Lt = 0.f, Ot = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = exp2f(sm[0][w][lane] - Mt);
      Lt += sm[1][w][lane] * a;
      Ot += sm[2][w][lane] * a;
    }
    out[(size_t)h * kD + d] = Ot / Lt;
  }
}

// ---- generic path -----------------------------------------------------------------

template <typename T>
__device__ __forceinline__ float widen(T x) {
  return (float)x;
}

// scores[h][t] = scale * (sum_i q_h[i] * K[t][kvh*d + i]), i ascending,
// separate multiply and add (attention.rs:1212-1239).
template <typename T>
__global__ __launch_bounds__(256) void generic_scores_kernel(const float* __restrict__ q,
                                                             const T* __restrict__ kl, int kv_dim,
                                                             int head_dim, int group, int positions,
                                                             int kv_lo, float scale,
                                                             float* __restrict__ scores) {
#pragma clang fp contract(off)
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int hr = blockIdx.y;  // q head within the range
  if (t >= positions) return;
  const int h = kv_lo * group + hr;
  const int kvh = h / group;
  const float* qh = q + (size_t)h * head_dim;
  const T* kr = kl + (size_t)t * kv_dim + (size_t)kvh * head_dim;
  float acc = 0.f;
  for (int i = 0; i < head_dim; ++i) acc += qh[i] * widen(kr[i]);
  scores[(size_t)hr * positions + t] = scale * acc;
}

// softmax over one head's scores (primitives/softmax.rs:18-40): max in f32,
// exp and sum in f64, multiply by the f32 reciprocal.
__global__ __launch_bounds__(256) void generic_softmax_kernel(float* __restrict__ scores, int positions) {
  float* x = scores + (size_t)blockIdx.x * positions;
  __shared__ float s_max[4];
  __shared__ double s_sum[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float mx = -INFINITY;
  for (int t = tid; t < positions; t += 256) mx = x[t] > mx ? x[t] : mx;
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(mx, off, 64);
    mx = o > mx ? o : mx;
  }
  if (lane == 0) s_max[wave] = mx;
  __syncthreads();
  mx = s_max[0];
  for (int w = 1; w < 4; ++w) mx = s_max[w] > mx ? s_max[w] : mx;
  const double m = (double)mx;
  double sum = 0.0;
  for (int t = tid; t < positions; t += 256) {
    const double e = exp((double)x[t] - m);
    x[t] = (float)e;
    sum += e;
  }
  sum = wave_sum_f64(sum);
  if (lane == 0) s_sum[wave] = sum;
  __syncthreads();
  sum = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
  const float inv = (float)(1.0 / sum);
  for (int t = tid; t < positions; t += 256) x[t] *= inv;
}

// out[h][i] = sum_t p[h][t] * V[t][kvh*d + i], t ascending (attention.rs:1278-1303).
template <typename T>
__global__ __launch_bounds__(64) void generic_vreduce_kernel(const float* __restrict__ p,
                                                             const T* __restrict__ vl, int kv_dim,
                                                             int head_dim, int group, int positions,
                                                             int kv_lo, float* __restrict__ out) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int hr = blockIdx.y;
  if (i >= head_dim) return;
  const int kvh = (kv_lo * group + hr) / group;
  const float* ph = p + (size_t)hr * positions;
  const T* vc = vl + (size_t)kvh * head_dim + i;
  float acc = 0.f;
  for (int t = 0; t < positions; ++t) acc += ph[t] * widen(vc[(size_t)t * kv_dim]);
  out[(size_t)hr * head_dim + i] = acc;
}

struct SplitArgs {
  const float* q;
  const void* kl;
  const void* vl;
  int kv_dim, positions, split_len, n_splits, n_units, group, n_hg, kv_lo;
  float qscale;
  float* part;
  float* out;
};

template <typename T, int G, int R, int W>
void launch_split(const SplitArgs& a, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.n_units + 7) / 8 * 8 * a.n_hg);
  hipLaunchKernelGGL((decode_split_kernel<T, G, R, W>), dim3(blocks), dim3(W * 64), 0, s, a.q, (const T*)a.kl,
                     (const T*)a.vl, a.kv_dim, a.positions, a.split_len, a.n_splits, a.n_units, a.group, a.n_hg,
                     a.kv_lo, a.qscale, a.part, a.out);
}

template <typename T, int G, int W>
void launch_split_r(const SplitArgs& a, hipStream_t s) {
  const int steps = a.split_len / (W * 4);
  if (steps >= 4 && G <= 4)  // G 8 x R 4 with ping-pong buffers would spill
    launch_split<T, G, 4, W>(a, s);
  else if (steps >= 2)
    launch_split<T, G, 2, W>(a, s);
  else
    launch_split<T, G, 1, W>(a, s);
}

template <typename T, int W>
void launch_split_g(int hg_size, const SplitArgs& a, hipStream_t s) {
  switch (hg_size) {
    case 1: launch_split_r<T, 1, W>(a, s); break;
    case 2: launch_split_r<T, 2, W>(a, s); break;
    case 4: launch_split_r<T, 4, W>(a, s); break;
    default: launch_split_r<T, 8, W>(a, s); break;
  }
}

}  // namespace

// Launch shape of the fast path: query heads per workgroup (the largest of
// 8/4/2/1 that divides the group and does not exceed the tuned size, default
// 2), waves per workgroup (default 4) and positions per split (default: about
// 512 workgroups in all, at least 64 positions each, at most kMaxSplits
// splits per kv head), rounded to the workgroup's row step.
struct DecodeShape {
  int hg_size, waves, split_len;
};

static DecodeShape pick_shape(const rv_kv* kv, int positions, int n_heads, int group) {
  DecodeShape d;
  const int want_hg = kv->tune_decode_hg > 0 ? (int)kv->tune_decode_hg : 2;
  d.hg_size = 1;
  for (int h : {8, 4, 2})
    if (h <= want_hg && group % h == 0) {
      d.hg_size = h;
      break;
    }
  d.waves = kv->tune_decode_waves == 4 ? 4 : 8;
  const int step = d.waves * 4;
  long len = kv->tune_decode_split_len;
  if (len <= 0) {
    // ~256 workgroups in all (measured best at ctx 4096, fp32: 16 splits of
    // 256 positions for each of 16 (kv head, pair of heads) jobs).
    const long jobs = (long)n_heads * (group / d.hg_size);
    const long splits = std::max<long>(1, 256 / jobs);
    len = std::max<long>(64, ((long)positions + splits - 1) / splits);
  }
  len = std::max<long>(len, ((long)positions + kMaxSplits - 1) / kMaxSplits);
  d.split_len = (int)((len + step - 1) / step * step);
  return d;
}

HipStatus launch_decode(rv_kv* kv, const float* q, size_t n_q_heads, size_t layer, size_t positions,
                        float scale, size_t kv_lo, size_t kv_hi, float* out, hipStream_t s) {
  HipStatus st;
  const int n_heads = (int)(kv_hi - kv_lo);
  if (n_heads == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const void* kl = kv->k_layer(layer);
  const void* vl = kv->v_layer(layer);
  // Kernel choice, from sweeps on MI355X: the MFMA kernel for f16 planes and
  // very long contexts (where it streams fastest), the VALU subgroup kernel
  // for fp32 planes up to 16K positions (where its shorter per-workgroup
  // critical path wins).
  const bool mfma = kv->tune_decode_impl == 2 ||
                    (kv->tune_decode_impl == 0 && (kv->elem == RV_ELEM_F16 || positions > 16384));
  if (kv->head_dim == kD && group <= 16 && mfma) {
    // MFMA path: ~512 positions per split (at least one 16-position tile per
    // wave), at most kMaxSplits splits.
    const int waves = kv->tune_decode_waves == 8 ? 8 : 4;
    const int step = waves * 16;
    long len = kv->tune_decode_split_len;
    if (len <= 0) len = std::max<long>(step, std::min<long>(512, ((long)positions * n_heads + 255) / 256));
    len = std::max<long>(len, ((long)positions + kMaxSplits - 1) / kMaxSplits);
    const int split_len = (int)((len + step - 1) / step * step);
    const int n_splits = (int)((positions + split_len - 1) / split_len);
    const size_t part_bytes = (size_t)n_heads * n_splits * part_stride_of(group) * sizeof(float);
    st = ensure_workspace(kv, part_bytes, 0);
    if (st.e != hipSuccess) return st;
    const dim3 grid((unsigned)(n_heads * n_splits));
    float* part = (float*)kv->ws;
    const float qscale = scale * kLog2e;
    if (kv->elem == RV_ELEM_F32) {
      if (waves == 4)
        hipLaunchKernelGGL((decode_mfma_kernel<float, 4>), grid, dim3(256), 0, s, q, (const float*)kl,
                           (const float*)vl, (int)kv->kv_dim, (int)positions, split_len, n_splits, group, (int)kv_lo,
                           qscale, part, out);
      else
        hipLaunchKernelGGL((decode_mfma_kernel<float, 8>), grid, dim3(512), 0, s, q, (const float*)kl,
                           (const float*)vl, (int)kv->kv_dim, (int)positions, split_len, n_splits, group, (int)kv_lo,
                           qscale, part, out);
    } else {
      if (waves == 4)
        hipLaunchKernelGGL((decode_mfma_kernel<_Float16, 4>), grid, dim3(256), 0, s, q, (const _Float16*)kl,
                           (const _Float16*)vl, (int)kv->kv_dim, (int)positions, split_len, n_splits, group,
                           (int)kv_lo, qscale, part, out);
      else
        hipLaunchKernelGGL((decode_mfma_kernel<_Float16, 8>), grid, dim3(512), 0, s, q, (const _Float16*)kl,
                           (const _Float16*)vl, (int)kv->kv_dim, (int)positions, split_len, n_splits, group,
                           (int)kv_lo, qscale, part, out);
    }
    if (n_splits > 1)
      hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)(n_heads * group * 2)), dim3(256), 0, s,
                         (const float*)part, n_splits, part_stride_of(group), group, group, 1, out);
  } else if (kv->head_dim == kD) {
    const DecodeShape d = pick_shape(kv, (int)positions, n_heads, group);
    const int n_hg = group / d.hg_size;
    const int n_splits = (int)((positions + d.split_len - 1) / d.split_len);
    const int n_jobs = n_heads * n_hg;
    const size_t part_bytes = (size_t)n_jobs * n_splits * part_stride_of(d.hg_size) * sizeof(float);
    st = ensure_workspace(kv, part_bytes, 0);
    if (st.e != hipSuccess) return st;
    SplitArgs a{q, kl, vl, (int)kv->kv_dim, (int)positions, d.split_len, n_splits, n_heads * n_splits, group,
                n_hg, (int)kv_lo, scale * kLog2e, (float*)kv->ws, out};
    if (kv->elem == RV_ELEM_F32) {
      if (d.waves == 4) launch_split_g<float, 4>(d.hg_size, a, s);
      else launch_split_g<float, 8>(d.hg_size, a, s);
    } else {
      if (d.waves == 4) launch_split_g<_Float16, 4>(d.hg_size, a, s);
      else launch_split_g<_Float16, 8>(d.hg_size, a, s);
    }
    if (n_splits > 1)
      hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)(n_jobs * d.hg_size * 2)), dim3(256), 0, s,
                         (const float*)kv->ws, n_splits, part_stride_of(d.hg_size), d.hg_size, group, n_hg, out);
  } else {
    const size_t hd = kv->head_dim;
    const int n_qr = n_heads * group;
    st = ensure_workspace(kv, (size_t)n_qr * positions * sizeof(float), 0);
    if (st.e != hipSuccess) return st;
    float* scores = (float*)kv->ws;
    const dim3 g1((unsigned)((positions + 255) / 256), (unsigned)n_qr);
    const dim3 g3((unsigned)((hd + 63) / 64), (unsigned)n_qr);
    if (kv->elem == RV_ELEM_F32) {
      hipLaunchKernelGGL(generic_scores_kernel<float>, g1, dim3(256), 0, s, q, (const float*)kl, (int)kv->kv_dim,
                         (int)hd, group, (int)positions, (int)kv_lo, scale, scores);
      hipLaunchKernelGGL(generic_softmax_kernel, dim3(n_qr), dim3(256), 0, s, scores, (int)positions);
      hipLaunchKernelGGL(generic_vreduce_kernel<float>, g3, dim3(64), 0, s, scores, (const float*)vl,
                         (int)kv->kv_dim, (int)hd, group, (int)positions, (int)kv_lo, out);
    } else {
      hipLaunchKernelGGL(generic_scores_kernel<_Float16>, g1, dim3(256), 0, s, q, (const _Float16*)kl,
                         (int)kv->kv_dim, (int)hd, group, (int)positions, (int)kv_lo, scale, scores);
      hipLaunchKernelGGL(generic_softmax_kernel, dim3(n_qr), dim3(256), 0, s, scores, (int)positions);
      hipLaunchKernelGGL(generic_vreduce_kernel<_Float16>, g3, dim3(64), 0, s, scores, (const _Float16*)vl,
                         (int)kv->kv_dim, (int)hd, group, (int)positions, (int)kv_lo, out);
    }
  }
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "decode launch";
  return st;
}

}  // namespace rv
