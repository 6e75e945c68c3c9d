// rv_decode.hip — single-token GQA decode attention on gfx950.
//
// Replaces attention_body / qk_scores / softmax / v_reduce
// (crates/core/src/kernels/attention.rs:1075-1303) for the decode and
// position-limited forms.
//
// Fast path (head_dim 128, group <= 16): decode_tile_kernel, one workgroup
// of W waves per (kv head, split of the position axis). The group's query
// heads are the columns of fp32 MFMA tiles over 16-position tiles of K and V,
// loaded straight into registers in the MFMA operand layouts; softmax is
// online (running max and sum per query head, exp2 with log2(e) folded into
// q). The splits of one kv head are merged by a second kernel with an fp32
// log-sum-exp combine. The kernel boundary is what makes the partials
// visible: the workgroups of one kv head run on different XCDs, whose L2s are
// not coherent, and an in-kernel hand-off would need agent-scope release and
// acquire fences (an L2 write-back and invalidate each), measured dearer
// than the second launch.
//
// VALU path (head_dim 128, any group; groups over 16 use it by default):
// decode_split_kernel, one workgroup per (kv head, subgroup of G query heads,
// split); a K or V row's head slice is read by one 16-lane group, 8 elements
// per lane, and serves the subgroup's G heads from registers; QK dots reduce
// over the 16 lanes with DPP. Same merge kernel.
//
// Generic path (any head_dim, any group): scores, softmax and the V
// reduction as three kernels in the reference's own order — f32 dots with
// i ascending and separate multiply/add, an f64 exp/sum softmax, and the V
// sum over t ascending per output element.
#include "rv_device.hpp"
#include "rv_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace rv {
namespace {

constexpr int kD = 128;                     // head_dim of the fast path
constexpr int kLPR = 16;                    // lanes per K/V row (8 elements each)
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
// grid numbers the n_hg subgroups of one (kv head, split) unit 8 apart, so
// they are dispatched in the same round and their repeated reads of the same
// K/V rows can hit in the shared cache levels. With one split the workgroup
// writes `out`; otherwise its partial (o, max, sum) row, merged by
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

// A plane element as the cache holds it: f32, or f16 bits with the
// reference's round-to-nearest-even (kv/mod.rs append).
template <typename T>
__device__ __forceinline__ void store_plane(T* p, float v);
template <>
__device__ __forceinline__ void store_plane<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_plane<_Float16>(_Float16* p, float v) {
  *reinterpret_cast<uint16_t*>(p) = f32_to_f16_bits(v);
}

// ---- MFMA path ----------------------------------------------------------------------

// 16-byte vector of plane elements: 4 fp32 or 8 f16.
template <typename T>
struct Chunk;
template <>
struct Chunk<float> {
  typedef f32x4 type;
  static constexpr int n = 4;
};
template <>
struct Chunk<_Float16> {
  typedef f16x8 type;
  static constexpr int n = 8;
};

// One workgroup of W waves per (kv head, split); the `group` (<= 16) query
// heads of the kv head are the 16 columns of fp32 MFMA tiles
// (v_mfma_f32_16x16x4_f32: exact fp32 products, fp32 accumulation). Wave w
// takes the split's 16-position tiles w, w+W, ...; every operand comes
// straight from global memory into registers, 16 bytes per load, in the
// layout the MFMA consumes, so nothing is staged through LDS:
//   S^T[t][m] = sum_d K[t][d] Q[m][d]: 32 MFMAs; lane (t, k) holds K row t
//     and lane (m, k) holds q head m at d = E*(k + 4*(s/E)) + s%E for step
//     s (E = elements per 16-byte chunk), i.e. chunks k, k+4, ... of the row;
//     log2(e)*scale is folded into q;
//   online softmax on the accumulator: lane l holds rows 4*(l/16) + r of
//     column l % 16, so a column's max needs two cross-lane swaps and every
//     exp is computed once;
//   O^T[d][m] += sum_t V[t][d] P^T[t][m]: 8 x 4 MFMAs; the accumulator layout
//     of S^T is exactly the B layout P^T needs (step r takes rows 4k + r), and
//     lane (i, k) holds V[4k + r][8i .. 8i+7], so output block b is d = 8i + b.
// The first tile's loads are issued before anything waits (a scheduling
// barrier keeps the compiler from sinking them to their uses), the next
// tile's after the current one is computed. The waves merge through LDS; the
// workgroup writes `out` (one split) or its partial (o, max, sum) row for
// decode_merge_kernel.
// With PRO the decode step's prologue runs here too (DecodePro): the planes
// are then written (the token's row) as well as read, so they are not
// declared __restrict__ (a restrict-qualified read-only plane would let the
// compiler treat its loads as unclobbered by the row's store).
struct NoPro {};
template <bool PRO, typename T>
using PlanePtr = std::conditional_t<PRO, const T*, const T* __restrict__>;

// H16 (f16 planes, no PRO): f16 MFMA operands (v_mfma_f32_16x16x16_f16)
// with fp32-equivalent products. K and V are exact in f16. Each head's q
// (scaled by a power of two so that its largest value is at most 2^14) is
// split into f16 hi + lo halves, and the scores scaled back exactly. The
// probabilities, scaled by 2^14 so that their low halves stay normal, are
// split the same way, and the output rescaled by 2^-14 at the end. Each MFMA
// takes 4 of the 8 values of a 16-byte K chunk (K·q: the same d slots from q)
// or element b of a lane's four V rows (P·V: the S^T accumulator is already
// the B layout), so the loads and the output layout are the fp32 path's.
template <typename T, int W, bool PRO = false, bool H16 = false>
__global__ __launch_bounds__(W * 64) void decode_tile_kernel(const float* __restrict__ q, PlanePtr<PRO, T> kl,
                                                             PlanePtr<PRO, T> vl, int kv_dim, int positions,
                                                             int split_len, int n_splits, int group, int kv_lo,
                                                             float qscale, float* __restrict__ part,
                                                             float* __restrict__ out,
                                                             std::conditional_t<PRO, DecodePro, NoPro> pro = {}) {
  typedef typename Chunk<T>::type CT;
  constexpr int E = Chunk<T>::n;
  constexpr int NKC = 32 / E;  // K chunks per lane per tile
  constexpr int NVC = 32 / E;  // V chunks per lane per tile (4 rows x 8 elements)
  constexpr int NT = W * 64;
  const int split = blockIdx.x % n_splits;
  const int hidx = blockIdx.x / n_splits;  // kv head within the range
  const int kvh = kv_lo + hidx;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lk = lane >> 4;
  const int t_begin = split * split_len;
  const int t_end = min(positions, t_begin + split_len);
  const int n_tiles = (t_end - t_begin + 15) / 16;
  const int my_tiles = n_tiles > wave ? (n_tiles - wave + W - 1) / W : 0;
  const size_t col = (size_t)kvh * kD;
  const bool col_ok = li < group;

  if constexpr (PRO) {
    // The token's row (position positions - 1) lives in the last split:
    // wave 0 writes this kv head's k (RMSNorm, then the rotation of pairs
    // (i, i + 64), as norm.rs:18-26 and rope.rs:31-45, contraction off) and
    // v into the cache row; the barrier makes them visible to the tiles.
    if (split == n_splits - 1) {
      if (wave == 0) {
#pragma clang fp contract(off)
        const float* kr = pro.k + col;
        const float* vr = pro.v + col;
        const float k0 = kr[lane], k1 = kr[lane + 64];
        const double ss = wave_sum_f64((double)k0 * (double)k0 + (double)k1 * (double)k1);
        const float inv = (float)(1.0 / sqrt(ss / (double)kD + (double)pro.eps));
        const float a0 = k0 * inv * pro.k_w[lane], a1 = k1 * inv * pro.k_w[lane + 64];
        const float c = pro.cs[lane], sn = pro.sn[lane];
        T* krow = const_cast<T*>(kl) + (size_t)(positions - 1) * kv_dim + col;
        T* vrow = const_cast<T*>(vl) + (size_t)(positions - 1) * kv_dim + col;
        store_plane<T>(krow + lane, a0 * c - a1 * sn);
        store_plane<T>(krow + lane + 64, a0 * sn + a1 * c);
        store_plane<T>(vrow + lane, vr[lane]);
        store_plane<T>(vrow + lane + 64, vr[lane + 64]);
      }
      __threadfence_block();
      __syncthreads();
    }
  }
  float qv[32];
  {
    // q may be only 4-byte aligned: scalar loads (once per workgroup).
    const float* qp = q + (size_t)(kvh * group + (col_ok ? li : 0)) * kD;
#pragma unroll
    for (int c = 0; c < NKC; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) qv[c * E + e] = qp[E * (lk + 4 * c) + e];
  }
  // Rows past the split re-read its last row (in bounds, branch-free); their
  // scores are masked below.
  auto load_tile = [&](int j, CT (&kb)[NKC], CT (&vb)[NVC]) {
    const int t0 = t_begin + (wave + j * W) * 16;
    const T* kp = kl + (size_t)min(t0 + li, t_end - 1) * kv_dim + col + E * lk;
#pragma unroll
    for (int c = 0; c < NKC; ++c) kb[c] = *reinterpret_cast<const CT*>(kp + 4 * E * c);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const T* vp = vl + (size_t)min(t0 + 4 * lk + r, t_end - 1) * kv_dim + col + 8 * li;
#pragma unroll
      for (int h = 0; h < 8 / E; ++h) vb[r * (8 / E) + h] = *reinterpret_cast<const CT*>(vp + E * h);
    }
  };
  // q is scaled once the first tile's loads are in flight (its own loads
  // then complete under theirs).
  const float qsc = col_ok ? qscale : 0.f;
  f16x4 qh[H16 ? 8 : 1], ql[H16 ? 8 : 1];
  float q_up = 1.f;
  auto scale_q = [&]() {
    if constexpr (PRO) {
#pragma clang fp contract(off)
      // RMSNorm of head li over its 128 values (this lane holds 32, the
      // lanes 16 and 32 apart the rest), then the rotation of pairs
      // (d, d + 64): chunks c and c + NKC / 2 of the same lane.
      double ss = 0.0;
#pragma unroll
      for (int i = 0; i < 32; ++i) ss += (double)qv[i] * (double)qv[i];
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      const float inv = (float)(1.0 / sqrt(ss / (double)kD + (double)pro.eps));
#pragma unroll
      for (int c = 0; c < NKC / 2; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int d = E * (lk + 4 * c) + e;  // < 64
          const float a0 = qv[c * E + e] * inv * pro.q_w[d];
          const float a1 = qv[(c + NKC / 2) * E + e] * inv * pro.q_w[d + 64];
          qv[c * E + e] = a0 * pro.cs[d] - a1 * pro.sn[d];
          qv[(c + NKC / 2) * E + e] = a0 * pro.sn[d] + a1 * pro.cs[d];
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) qv[i] *= qsc;
    if constexpr (H16) {
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(qv[i]));
      amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
      int ex = 0;
      (void)frexpf(amax, &ex);  // amax < 2^ex
      const int k = ex > 14 ? ex - 14 : 0;
      const float down = ldexpf(1.f, -k);
      q_up = ldexpf(1.f, k);
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const float v = qv[(m >> 1) * 8 + 4 * (m & 1) + kk] * down;
          const _Float16 h = (_Float16)v;
          qh[m][kk] = h;
          ql[m][kk] = (_Float16)(v - (float)h);
        }
    }
  };

  f32x4 o[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegSentinel, l_run = 0.f;
  auto compute = [&](int j, const CT (&kb)[NKC], const CT (&vb)[NVC]) {
    const int t0 = t_begin + (wave + j * W) * 16;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (H16) {
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const f16x4 k4 = {(_Float16)kb[m >> 1][4 * (m & 1)], (_Float16)kb[m >> 1][4 * (m & 1) + 1],
                          (_Float16)kb[m >> 1][4 * (m & 1) + 2], (_Float16)kb[m >> 1][4 * (m & 1) + 3]};
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(k4, qh[m], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(k4, ql[m], acc, 0, 0, 0);
      }
      acc *= q_up;
    } else {
#pragma unroll
      for (int c = 0; c < NKC; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32((float)kb[c][e], qv[c * E + e], acc, 0, 0, 0);
    }
    float x[4], mx = kNegSentinel;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = (t0 + 4 * lk + r < t_end) ? acc[r] : -INFINITY;
      mx = fmaxf(mx, x[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m_run, mx);
    // v_exp_f32 directly: results below 2^-126 flush to zero, which only
    // drops weights that are negligible next to the running maximum's 1.
    const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
    m_run = mn;
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(x[r] - mn);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    if constexpr (H16) {
      f16x4 ph, pl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pp = p[r] * 16384.f;
        const _Float16 h = (_Float16)pp;
        ph[r] = h;
        pl[r] = (_Float16)(pp - (float)h);
      }
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        o[b] *= alpha;
        const f16x4 v4 = {(_Float16)vb[0][b], (_Float16)vb[1][b], (_Float16)vb[2][b], (_Float16)vb[3][b]};
        o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(v4, ph, o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(v4, pl, o[b], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        o[b] *= alpha;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)vb[(r * 8 + b) / E][(r * 8 + b) % E], p[r], o[b], 0, 0, 0);
      }
    }
  };
  // Every load of a tile is issued unconditionally before the tile is used
  // (exact wait counts: its first MFMAs start as its first chunks land); the
  // sched_barrier keeps the compiler from sinking them to their first use.
  // 4-wave workgroups take tiles in pairs (two in flight per wave); 8-wave
  // ones one at a time, keeping their registers within four waves per SIMD.
  CT ka[NKC], va[NVC];
  int j = 0;
  if constexpr (W == 4) {
    CT kb2[NKC], vb2[NVC];
    for (; j + 1 < my_tiles; j += 2) {
      load_tile(j, ka, va);
      load_tile(j + 1, kb2, vb2);
      __builtin_amdgcn_sched_barrier(0);
      if (j == 0) scale_q();
      compute(j, ka, va);
      compute(j + 1, kb2, vb2);
    }
  }
  for (; j < my_tiles; ++j) {
    load_tile(j, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    if (j == 0) scale_q();
    compute(j, ka, va);
  }
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  if constexpr (H16) {
#pragma unroll
    for (int b = 0; b < 8; ++b) o[b] *= 1.f / 16384.f;  // the probabilities' 2^14, exactly
  }
  // o[b][r] = O^T[d = 8*(4*lk + r) + b][m = li]. Merge the W waves in LDS.
  __shared__ __attribute__((aligned(16))) float sm_o[W][16][kD + 4];
  __shared__ float sm_ml[W][16][2];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float* dst = &sm_o[wave][li][8 * (4 * lk + r)];
    *reinterpret_cast<f32x4*>(dst) = f32x4{o[0][r], o[1][r], o[2][r], o[3][r]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o[4][r], o[5][r], o[6][r], o[7][r]};
  }
  if (lk == 0) {
    sm_ml[wave][li][0] = m_run;
    sm_ml[wave][li][1] = l_run;
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
      const float a = __builtin_amdgcn_exp2f(sm_ml[w][g][0] - M);
      L += sm_ml[w][g][1] * a;
      O += *reinterpret_cast<const f32x4*>(&sm_o[w][g][d]) * a;
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
// heads) partial row set: one 256-thread workgroup per (query head, block of
// kMergeCols output columns), its threads a grid of 256/kMergeCols split
// lanes x kMergeCols columns. Each thread loads a chunk of kMergeChunk splits
// (o, max, sum) before it folds any of them, so a chunk costs one memory
// round trip; the split lanes then merge through LDS.
constexpr int kMergeCols = 32;
constexpr int kMergeChunk = 8;
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part, int n_splits, int stride,
                                                           int G, int group, int n_hg, float* __restrict__ out) {
  constexpr int NS = 256 / kMergeCols;
  constexpr int NB = kD / kMergeCols;
  const int blk = blockIdx.x % NB, jg = blockIdx.x / NB;
  const int g = jg % G, job = jg / G;
  const int hidx = job / n_hg, hg = job % n_hg;
  const int h = hidx * group + hg * G + g;  // q head within the range
  const int tid = threadIdx.x, ci = tid % kMergeCols, sl = tid / kMergeCols;
  const int d = blk * kMergeCols + ci;
  const float* base = part + (size_t)job * n_splits * stride;
  float M = kNegSentinel, L = 0.f, O = 0.f;
  for (int b0 = 0; b0 < n_splits; b0 += NS * kMergeChunk) {
    float ov[kMergeChunk], mv[kMergeChunk], lv[kMergeChunk];
#pragma unroll
    for (int i = 0; i < kMergeChunk; ++i) {
      const float* ps = base + (size_t)min(b0 + NS * i + sl, n_splits - 1) * stride;
      ov[i] = ps[g * kD + d];
      mv[i] = ps[G * kD + 2 * g];
      lv[i] = ps[G * kD + 2 * g + 1];
    }
    float mc = M;
#pragma unroll
    for (int i = 0; i < kMergeChunk; ++i)
      if (b0 + NS * i + sl < n_splits) mc = fmaxf(mc, mv[i]);
    const float a = __builtin_amdgcn_exp2f(M - mc);
    L *= a;
    O *= a;
#pragma unroll
    for (int i = 0; i < kMergeChunk; ++i)
      if (b0 + NS * i + sl < n_splits) {
        const float c = __builtin_amdgcn_exp2f(mv[i] - mc);
        L += lv[i] * c;
        O += ov[i] * c;
      }
    M = mc;
  }
  __shared__ float sm[3][NS][kMergeCols + 1];
  sm[0][sl][ci] = M;
  sm[1][sl][ci] = L;
  sm[2][sl][ci] = O;
  __syncthreads();
  if (tid < kMergeCols) {
    float Mt = sm[0][0][tid];
#pragma unroll
    for (int i = 1; i < NS; ++i) Mt = fmaxf(Mt, sm[0][i][tid]);
    float Lt = 0.f, Ot = 0.f;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const float a = __builtin_amdgcn_exp2f(sm[0][i][tid] - Mt);
      Lt += sm[1][i][tid] * a;
      Ot += sm[2][i][tid] * a;
    }
    out[(size_t)h * kD + blk * kMergeCols + tid] = Ot / Lt;
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
  TimedPair tp;
};

template <typename T, int G, int R, int W>
void launch_split(const SplitArgs& a, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.n_units + 7) / 8 * 8 * a.n_hg);
  launch_timed(a.tp, decode_split_kernel<T, G, R, W>, dim3(blocks), dim3(W * 64), s, a.q, (const T*)a.kl,
               (const T*)a.vl, a.kv_dim, a.positions, a.split_len, a.n_splits, a.n_units, a.group, a.n_hg, a.kv_lo,
               a.qscale, a.part, a.out);
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

// Launch shape of the VALU subgroup path: query heads per workgroup (the
// largest of 8/4/2/1 that divides the group and does not exceed the tuned
// size, default 2), waves per workgroup (default 8) and positions per split
// (default: about 256 workgroups in all, at least 64 positions each), rounded
// to the workgroup's row step.
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
    const long jobs = (long)n_heads * (group / d.hg_size);
    const long splits = std::max<long>(1, 256 / jobs);
    len = std::max<long>(64, ((long)positions + splits - 1) / splits);
  }
  d.split_len = (int)((len + step - 1) / step * step);
  return d;
}

static void launch_merge(const float* part, int n_splits, int G, int group, int n_hg, int n_q, float* out,
                         hipStream_t s) {
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)(n_q * (kD / kMergeCols))), dim3(256), 0, s, part, n_splits,
                     part_stride_of(G), G, group, n_hg, out);
}

template <typename T, bool H16 = false>
static void launch_tile(const TimedPair& tp, int waves, dim3 grid, hipStream_t s, const float* q, const void* kl,
                        const void* vl, int kv_dim, int positions, int split_len, int n_splits, int group, int kv_lo,
                        float qscale, float* part, float* out) {
  if (waves == 8)
    launch_timed(tp, decode_tile_kernel<T, 8, false, H16>, grid, dim3(512), s, q, (const T*)kl, (const T*)vl, kv_dim,
                 positions, split_len, n_splits, group, kv_lo, qscale, part, out, NoPro{});
  else
    launch_timed(tp, decode_tile_kernel<T, 4, false, H16>, grid, dim3(256), s, q, (const T*)kl, (const T*)vl, kv_dim,
                 positions, split_len, n_splits, group, kv_lo, qscale, part, out, NoPro{});
}

bool decode_pro_supported(const rv_kv* kv, size_t n_q_heads) {
  return kv->head_dim == kD && n_q_heads % kv->n_kv_heads == 0 && n_q_heads / kv->n_kv_heads <= 16 &&
         kv->tune_decode_impl != 1;
}

HipStatus launch_decode_pro(rv_kv* kv, const float* q_raw, size_t n_q_heads, size_t layer, size_t positions,
                            float scale, const DecodePro& pro, float* out, hipStream_t s) {
  HipStatus st;
  const int n_heads = (int)kv->n_kv_heads;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  // The launch shape of launch_decode's MFMA path.
  const long want = ((long)positions * n_heads + 511) / 512;
  const int waves = kv->tune_decode_waves == 8 || kv->tune_decode_waves == 4 ? (int)kv->tune_decode_waves
                                                                             : (want >= 256 ? 8 : 4);
  const int step = waves * 16;
  long len = kv->tune_decode_split_len;
  if (len <= 0) len = want;
  len = std::max<long>(len, step);
  const int split_len = (int)((len + step - 1) / step * step);
  const int n_splits = (int)((positions + split_len - 1) / split_len);
  st = ensure_workspace(kv, (size_t)n_heads * n_splits * part_stride_of(group) * sizeof(float));
  if (st.e != hipSuccess) return st;
  float* part = (float*)kv->ws;
  const dim3 grid((unsigned)(n_heads * n_splits));
  const TimedPair tp = timing_pair(kv, s);
  const float qscale = scale * kLog2e;
  auto go = [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    const T* kl = (const T*)kv->k_layer(layer);
    const T* vl = (const T*)kv->v_layer(layer);
    if (waves == 8)
      launch_timed(tp, decode_tile_kernel<T, 8, true>, grid, dim3(512), s, q_raw, kl, vl, (int)kv->kv_dim,
                   (int)positions, split_len, n_splits, group, 0, qscale, part, out, pro);
    else
      launch_timed(tp, decode_tile_kernel<T, 4, true>, grid, dim3(256), s, q_raw, kl, vl, (int)kv->kv_dim,
                   (int)positions, split_len, n_splits, group, 0, qscale, part, out, pro);
  };
  if (kv->elem == RV_ELEM_F32)
    go((float*)nullptr);
  else
    go((_Float16*)nullptr);
  if (n_splits > 1) launch_merge(part, n_splits, group, group, 1, n_heads * group, out, s);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "decode launch";
  return st;
}

HipStatus launch_decode(rv_kv* kv, const float* q, size_t n_q_heads, size_t layer, size_t positions,
                        float scale, size_t kv_lo, size_t kv_hi, float* out, hipStream_t s) {
  HipStatus st;
  const int n_heads = (int)(kv_hi - kv_lo);
  if (n_heads == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const void* kl = kv->k_layer(layer);
  const void* vl = kv->v_layer(layer);
  const float qscale = scale * kLog2e;
  if (kv->head_dim == kD && group <= 16 && kv->tune_decode_impl != 1) {
    // MFMA tile kernel. Default shape, from sweeps on MI355X: about 512
    // workgroups in all, 4 waves (one tile each, 64 positions at ctx 4096)
    // while splits stay short, 8 waves from 256 positions per split (ctx
    // 32768: two tiles per wave); never less than one tile per wave.
    const long want = ((long)positions * n_heads + 511) / 512;
    const int waves = kv->tune_decode_waves == 8 || kv->tune_decode_waves == 4 ? (int)kv->tune_decode_waves
                                                                               : (want >= 256 ? 8 : 4);
    const int step = waves * 16;
    long len = kv->tune_decode_split_len;
    if (len <= 0) len = want;
    len = std::max<long>(len, step);
    const int split_len = (int)((len + step - 1) / step * step);
    const int n_splits = (int)((positions + split_len - 1) / split_len);
    st = ensure_workspace(kv, (size_t)n_heads * n_splits * part_stride_of(group) * sizeof(float));
    if (st.e != hipSuccess) return st;
    float* part = (float*)kv->ws;
    const dim3 grid((unsigned)(n_heads * n_splits));
    const TimedPair tp = timing_pair(kv, s);
    if (kv->elem == RV_ELEM_F32)
      launch_tile<float>(tp, waves, grid, s, q, kl, vl, (int)kv->kv_dim, (int)positions, split_len, n_splits, group,
                         (int)kv_lo, qscale, part, out);
    else if (kv->tune_decode_impl == 2)  // fp32 MFMA operands for f16 planes (the reference form)
      launch_tile<_Float16>(tp, waves, grid, s, q, kl, vl, (int)kv->kv_dim, (int)positions, split_len, n_splits, group,
                            (int)kv_lo, qscale, part, out);
    else
      launch_tile<_Float16, true>(tp, waves, grid, s, q, kl, vl, (int)kv->kv_dim, (int)positions, split_len, n_splits,
                                  group, (int)kv_lo, qscale, part, out);
    if (n_splits > 1) launch_merge(part, n_splits, group, group, 1, n_heads * group, out, s);
  } else if (kv->head_dim == kD) {
    const DecodeShape d = pick_shape(kv, (int)positions, n_heads, group);
    const int n_hg = group / d.hg_size;
    const int n_splits = (int)((positions + d.split_len - 1) / d.split_len);
    const int n_jobs = n_heads * n_hg;
    const size_t part_bytes = (size_t)n_jobs * n_splits * part_stride_of(d.hg_size) * sizeof(float);
    st = ensure_workspace(kv, part_bytes);
    if (st.e != hipSuccess) return st;
    SplitArgs a{q, kl, vl, (int)kv->kv_dim, (int)positions, d.split_len, n_splits, n_heads * n_splits, group,
                n_hg, (int)kv_lo, qscale, (float*)kv->ws, out, timing_pair(kv, s)};
    if (kv->elem == RV_ELEM_F32) {
      if (d.waves == 4) launch_split_g<float, 4>(d.hg_size, a, s);
      else launch_split_g<float, 8>(d.hg_size, a, s);
    } else {
      if (d.waves == 4) launch_split_g<_Float16, 4>(d.hg_size, a, s);
      else launch_split_g<_Float16, 8>(d.hg_size, a, s);
    }
    if (n_splits > 1) launch_merge((const float*)kv->ws, n_splits, d.hg_size, group, n_hg, n_jobs * d.hg_size, out, s);
  } else {
    const size_t hd = kv->head_dim;
    const int n_qr = n_heads * group;
    st = ensure_workspace(kv, (size_t)n_qr * positions * sizeof(float));
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
