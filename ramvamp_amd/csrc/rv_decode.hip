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
// log-sum-exp combine (decode_merge_kernel), or inside the tile launch (the
// XCD merge: the splits that share an XCD fold in its L2, then one row per
// XCD crosses), a tuning option that measured slower at the headline shape
// (its two acknowledged stores and two atomic round trips in series cost
// more than the second launch).
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
#include <mutex>
#include <type_traits>

namespace rv {
namespace {

constexpr int kD = 128;                     // head_dim of the fast path
constexpr int kLPR = 16;                    // lanes per K/V row (8 elements each)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegSentinel = -1.0e30f;    // finite "no position yet" max
// Decode softmax: scores (log2 units) may exceed the running maximum by up to
// kSlack before it moves, so probabilities are at most 2^kSlack; the f16 path
// splits p * kPScale (<= 2^14, inside f16's range) into hi + lo halves.
constexpr float kSlack = 8.f;
constexpr float kPScale = 64.f;

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
// Each wave keeps D tiles in flight in a register ring (D = 1 when the grid
// holds two waves per SIMD):
// the first D tiles' loads are issued before anything waits, and the loads
// of tile j + D are issued as soon as tile j has been computed (scheduling
// barriers keep the compiler from sinking them to their first use). The
// kernel is held to 256 registers so that two waves fit per SIMD and a grid
// of ~2048 waves is resident at once. The waves merge through LDS; the workgroup then writes
// `out` (one split) or its partial (o, max, sum) row; the splits of a kv head
// are folded by decode_merge_kernel or, in MergeMode kMergeXcd, inside the
// same launch (the in-launch split merge below).
// With PRO the decode step's prologue runs here too (DecodePro): the planes
// are then written (the token's row) as well as read, so they are not
// declared __restrict__ (a restrict-qualified read-only plane would let the
// compiler treat its loads as unclobbered by the row's store).
struct NoPro {};
template <bool PRO, typename T>
using PlanePtr = std::conditional_t<PRO, const T*, const T* __restrict__>;

// ---- in-launch split merge (the XCD merge) ----------------------------------------------
// The dispatcher deals a launch's workgroups to the 8 XCDs round robin, so
// workgroups whose indices agree mod 8 share an XCD and its L2 (the physical
// XCD of a slot changes between launches; the grouping does not). The L2s of
// different XCDs are not kept coherent with each other for ordinary stores.
// Level 1: the splits of a kv head with s = r (mod 8) share slot r's L2;
// each writes its partial row with plain stores, waits until they are
// complete (vmcnt 0), and takes a ticket; the last of the group folds the
// group's rows (loads that skip the CU's L1 and read that L2) in split order.
// Level 2: the group's row is written with device-scope (sc1) stores, which
// the L2 writes through; after a second ticket the last of the <= 8 groups
// folds their rows with device-scope loads, in group order. Each last
// arriver resets its ticket for the next call; no L2 write-back or
// invalidate is needed, and no workgroup waits on another. The fold order
// depends only on n_splits, so every kv head's result (and a kv-head range's)
// is the same whichever workgroups finish last.
constexpr int kPolicyDevice = 16;  // the sc1 bit of the buffer instructions' cache policy
constexpr int kPolicyL2 = 1;       // the sc0 bit: the load misses the CU's L1 and reads its XCD's L2

// How the splits of a kv head are folded.
enum MergeMode : int {
  kMergeKernel = 0,  // partials only; decode_merge_kernel folds them in a second launch
  kMergeXcd = 1,     // in-launch: a first level inside each XCD's L2, then one row per XCD across
};

struct MergeArgs {
  float* part;         // [n_heads][n_splits][stride], then [n_heads][8] level-2 rows
  unsigned* xt;        // counter (slot, head) at line slot * xpad + head, level 2 at line 8 * xpad + head
  uint32_t ws_bytes;   // bytes addressable from `part` (the buffer accesses' bound)
  int xpad;            // kv heads of the cache (lines per XCD slot)
  int mode;            // MergeMode
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(float* base, uint32_t bytes) {
  // Raw buffer over the workspace: stride 0, num_records in bytes (accesses
  // past it read 0 and drop their writes), the gfx9 data-format word.
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Folds `cnt` partial rows (o[group][kD], then (max, sum) per head),
// starting `row0` rows into the buffer, in row order: thread -> (head g, 4
// consecutive d). Writes a partial row at dst_row (when out is null) or the
// normalised output out[g * kD + d].
// Rows row0, row0 + step, ...; loaded with cache policy LP (device scope for
// rows other XCDs wrote, L2 for rows this XCD wrote); a partial row out is
// stored at device scope.
template <int NT, int LP = kPolicyDevice>
__device__ void fold_rows(__amdgpu_buffer_rsrc_t rs, uint32_t row0, int cnt, int stride, int group, uint32_t dst_row,
                          float* out, int tid, uint32_t step = 1) {
  constexpr int kChunk = 8;
  for (int j = tid; j < group * (kD / 4); j += NT) {
    const int g = j / (kD / 4), d = (j % (kD / 4)) * 4;
    float M = kNegSentinel, L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    for (int b0 = 0; b0 < cnt; b0 += kChunk) {
      f32x4 ov[kChunk];
      float mv[kChunk], lv[kChunk];
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const uint32_t row = (row0 + step * (uint32_t)min(b0 + i, cnt - 1)) * (uint32_t)stride * 4u;
        ov[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, row + (uint32_t)(g * kD + d) * 4u, 0, LP);
        mv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              rs, row + (uint32_t)(group * kD + 2 * g) * 4u, 0, LP));
        lv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              rs, row + (uint32_t)(group * kD + 2 * g + 1) * 4u, 0, LP));
      }
      float mc = M;
#pragma unroll
      for (int i = 0; i < kChunk; ++i)
        if (b0 + i < cnt) mc = fmaxf(mc, mv[i]);
      const float a = __builtin_amdgcn_exp2f(M - mc);
      L *= a;
      O *= a;
#pragma unroll
      for (int i = 0; i < kChunk; ++i)
        if (b0 + i < cnt) {
          const float c = __builtin_amdgcn_exp2f(mv[i] - mc);
          L += lv[i] * c;
          O += ov[i] * c;
        }
      M = mc;
    }
    if (out) {
      const f32x4 r = O / L;  // out may be only 4-byte aligned
      float* op = out + (size_t)g * kD + d;
      op[0] = r[0];
      op[1] = r[1];
      op[2] = r[2];
      op[3] = r[3];
    } else {
      const uint32_t row = dst_row * (uint32_t)stride * 4u;
      __builtin_amdgcn_raw_buffer_store_b128(O, rs, row + (uint32_t)(g * kD + d) * 4u, 0, kPolicyDevice);
      if (d == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, M), rs, row + (uint32_t)(group * kD + 2 * g) * 4u,
                                              0, kPolicyDevice);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, L), rs,
                                              row + (uint32_t)(group * kD + 2 * g + 1) * 4u, 0, kPolicyDevice);
      }
    }
  }
}

// Takes this workgroup's ticket on `t` once all its threads' partial stores
// are complete; true for the workgroup that drew the last of `n` tickets,
// which also resets the counter for the next call.
// The counter is device-wide (an agent-scope atomic: gfx950 issues the same
// instruction for workgroup scope, and it is coherent across XCDs).
__device__ __forceinline__ bool last_of(unsigned* t, unsigned n, int tid) {
  __shared__ unsigned sm_ticket;
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    const unsigned got = __hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (got == n - 1) __hip_atomic_store(t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm_ticket = got;
  }
  __syncthreads();
  return sm_ticket == n - 1;
}

// H16 (f16 planes, no PRO): f16 MFMA operands with fp32-equivalent
// products. K and V are exact in f16. Each head's q (scaled by a power of
// two so that its largest value is at most 2^14) is split into f16 hi + lo
// halves, and the scores scaled back exactly; K·q runs on
// v_mfma_f32_16x16x32_f16, whose A operand is a lane's loaded 16-byte K
// chunk as is (the same d slots of q as B). The probabilities, scaled by
// kPScale, are split the same way for P·V (v_mfma_f32_16x16x16_f16 on
// element b of a lane's four V rows: the S^T accumulator is already the B
// layout), and the output scaled back at the end; so the loads and the
// output layout are the fp32 path's.
template <typename T, int W, int D, bool PRO = false, bool H16 = false, bool LDS = false>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2))) void decode_tile_kernel(
    const float* __restrict__ q, PlanePtr<PRO, T> kl, PlanePtr<PRO, T> vl, int kv_dim, int positions, int split_len,
    int n_splits, int group, int kv_lo, float qscale, MergeArgs mg, float* __restrict__ out,
    std::conditional_t<PRO, DecodePro, NoPro> pro = {}) {
  typedef typename Chunk<T>::type CT;
  constexpr int E = Chunk<T>::n;
  constexpr int NKC = 32 / E;  // K chunks per lane per tile
  constexpr int NVC = 32 / E;  // V chunks per lane per tile (4 rows x 8 elements)
  constexpr int NT = W * 64;
  // The LDS form stages 64-position tiles (16 positions per wave) of K and V
  // for the whole workgroup, two stages of kStage bytes; the waves' merge
  // below reuses the same bytes once the ring is drained.
  static_assert(!LDS || (W == 4 && D == 1 && !PRO), "LDS staging: 4 waves, one tile per step, no prologue");
  constexpr int kRowB = kD * (int)sizeof(T);  // bytes of one position's head slice
  constexpr int kPlaneB = 64 * kRowB;         // one plane of a staged tile
  constexpr int kStage = 2 * kPlaneB;
  constexpr int kOBytes = W * 16 * (kD + 4) * (int)sizeof(float);
  constexpr int kLdsBytes = LDS ? (2 * kStage > kOBytes ? 2 * kStage : kOBytes) : kOBytes;
  __shared__ __attribute__((aligned(1024))) char lds_raw[kLdsBytes];
  if constexpr (PRO) {
    // A token graph's step: the token's position from device memory. One
    // past the plan is refused (as append refuses a full layer): no row is
    // written, `out` is left as it was, and the first refusal is recorded.
    if (pro.d_pos) {
      const uint32_t p = *pro.d_pos;
      if (p > (uint32_t)pro.max_pos) {
        if (blockIdx.x == 0 && threadIdx.x == 0 && pro.status[0] == 0) {
          pro.status[1] = pro.layer;
          pro.status[2] = p;
          pro.status[3] = (uint32_t)pro.max_pos + 1;
          pro.status[0] = RV_KV_CAPACITY_EXCEEDED;
        }
        return;
      }
      positions = (int)p + 1;
    }
  }
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
    // The token's row (position positions - 1) lives in the split that
    // holds it (the last one unless a token graph planned for more):
    // wave 0 writes this kv head's k (RMSNorm, then the rotation of pairs
    // (i, i + 64), as norm.rs:18-26 and rope.rs:31-45, contraction off) and
    // v into the cache row; the barrier makes them visible to the tiles.
    if (split == (positions - 1) / split_len) {
      if (wave == 0) {
#pragma clang fp contract(off)
        const float* kr = pro.k + col;
        const float* vr = pro.v + col;
        const float k0 = kr[lane], k1 = kr[lane + 64];
        const double ss = wave_sum_f64((double)k0 * (double)k0 + (double)k1 * (double)k1);
        const float inv = (float)(1.0 / sqrt(ss / (double)kD + (double)pro.eps));
        const float a0 = k0 * inv * pro.k_w[lane], a1 = k1 * inv * pro.k_w[lane + 64];
        const float* trow = pro.tab + (size_t)(positions - 1) * kD;
        const float c = pro.d_pos ? trow[lane] : pro.cs[lane], sn = pro.d_pos ? trow[64 + lane] : pro.sn[lane];
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
    // q may be only 4-byte aligned: scalar loads (once per workgroup). (Staging
    // the group's rows through LDS with coalesced loads measured slower: its
    // barrier costs more than the gather.)
    const float* qp = q + (size_t)(kvh * group + (col_ok ? li : 0)) * kD;
#pragma unroll
    for (int c = 0; c < NKC; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) qv[c * E + e] = qp[E * (lk + 4 * c) + e];
  }
  // Rows past the split re-read its last row (in bounds, branch-free); their
  // scores are masked below, and tiles past the wave's share are loaded that
  // way but never computed. K and V are read once per call: non-temporal
  // loads (config 2: 0.13 µs per call faster than plain loads).
  auto load_tile = [&](int j, CT (&kb)[NKC], CT (&vb)[NVC]) {
    const int t0 = t_begin + (wave + j * W) * 16;
    const T* kp = kl + (size_t)min(t0 + li, t_end - 1) * kv_dim + col + E * lk;
#pragma unroll
    for (int c = 0; c < NKC; ++c) kb[c] = __builtin_nontemporal_load(reinterpret_cast<const CT*>(kp + 4 * E * c));
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const T* vp = vl + (size_t)min(t0 + 4 * lk + r, t_end - 1) * kv_dim + col + 8 * li;
#pragma unroll
      for (int h = 0; h < 8 / E; ++h)
        vb[r * (8 / E) + h] = __builtin_nontemporal_load(reinterpret_cast<const CT*>(vp + E * h));
    }
  };
  // q is scaled once the first tiles' loads are in flight (its own loads
  // then complete under theirs).
  const float qsc = col_ok ? qscale : 0.f;
  f16x8 qh[H16 ? 4 : 1], ql[H16 ? 4 : 1];
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
      ss = swap_sum_f64<16>(ss);
      ss = swap_sum_f64<32>(ss);
      const float inv = (float)(1.0 / sqrt(ss / (double)kD + (double)pro.eps));
      const float* trow = pro.tab + (size_t)(positions - 1) * kD;
#pragma unroll
      for (int c = 0; c < NKC / 2; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int d = E * (lk + 4 * c) + e;  // < 64
          const float a0 = qv[c * E + e] * inv * pro.q_w[d];
          const float a1 = qv[(c + NKC / 2) * E + e] * inv * pro.q_w[d + 64];
          const float cs = pro.d_pos ? trow[d] : pro.cs[d], sn = pro.d_pos ? trow[64 + d] : pro.sn[d];
          qv[c * E + e] = a0 * cs - a1 * sn;
          qv[(c + NKC / 2) * E + e] = a0 * sn + a1 * cs;
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) qv[i] *= qsc;
    if constexpr (H16) {
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(qv[i]));
      amax = swap_max<16>(amax);
      amax = swap_max<32>(amax);
      int ex = 0;
      (void)frexpf(amax, &ex);  // amax < 2^ex
      const int k = ex > 14 ? ex - 14 : 0;
      const float down = ldexpf(1.f, -k);
      q_up = ldexpf(1.f, k);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = qv[c * 8 + e] * down;
          const _Float16 h = (_Float16)v;
          qh[c][e] = h;
          ql[c][e] = (_Float16)(v - (float)h);
        }
    }
  };

  f32x4 o[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegSentinel, l_run = 0.f;
  auto compute = [&](int j, const CT (&kb)[NKC], const CT (&vb)[NVC]) {
    const int t0 = t_begin + (wave + j * W) * 16;
    // Independent accumulator chains: a dependent MFMA waits for its
    // predecessor's result (~50 cycles on gfx950) where independent ones
    // issue every 16-32.
    f32x4 acc;
    if constexpr (H16) {
      // v_mfma_f32_16x16x32_f16: lane (t, k) supplies K[t][32c + 8k .. +7],
      // i.e. its loaded chunk c as is, and q the same slots; hi and lo
      // products in separate chains.
      f32x4 a4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        a4[2 * (c & 1)] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[c], qh[c], a4[2 * (c & 1)], 0, 0, 0);
        a4[2 * (c & 1) + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[c], ql[c], a4[2 * (c & 1) + 1], 0, 0, 0);
      }
      acc = ((a4[0] + a4[2]) + (a4[1] + a4[3])) * q_up;
    } else {
      f32x4 a4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NKC; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e)
          a4[e & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)kb[c][e], qv[c * E + e], a4[e & 3], 0, 0, 0);
      acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
    }
    float x[4], mx = kNegSentinel;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = (t0 + 4 * lk + r < t_end) ? acc[r] : -INFINITY;
      mx = fmaxf(mx, x[r]);
    }
    mx = swap_max<16>(mx);
    mx = swap_max<32>(mx);
    // Lazy rescaling: the running maximum (per query head) moves only when
    // a tile's scores exceed it by more than 2^kSlack, so the probabilities
    // stay within 2^kSlack and the accumulators are rescaled only then (a
    // wave-uniform branch, rare after a wave's first tile) instead of on
    // every tile, where the multiplies also stalled the PV MFMA chains.
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kSlack) != 0) {
      const float mn = fmaxf(m_run, mx);
      // v_exp_f32 directly: results below 2^-126 flush to zero, which only
      // drops weights negligible next to the running maximum's.
      const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
      m_run = mn;
      l_run *= alpha;
#pragma unroll
      for (int b = 0; b < 8; ++b) o[b] *= alpha;
    }
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(x[r] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
    // PV with consecutive MFMAs on different accumulators (a dependent MFMA
    // waits ~50 cycles for its predecessor).
    if constexpr (H16) {
      f16x4 ph, pl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pp = p[r] * kPScale;
        const _Float16 h = (_Float16)pp;
        ph[r] = h;
        pl[r] = (_Float16)(pp - (float)h);
      }
      f16x4 v4[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) v4[b] = f16x4{(_Float16)vb[0][b], (_Float16)vb[1][b], (_Float16)vb[2][b], (_Float16)vb[3][b]};
#pragma unroll
      for (int b = 0; b < 8; ++b) o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(v4[b], ph, o[b], 0, 0, 0);
#pragma unroll
      for (int b = 0; b < 8; ++b) o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(v4[b], pl, o[b], 0, 0, 0);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int b = 0; b < 8; ++b)
          o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32((float)vb[(r * 8 + b) / E][(r * 8 + b) % E], p[r], o[b], 0, 0, 0);
    }
  };
  // The ring: every load of a tile is issued unconditionally (exact wait
  // counts: a tile's first MFMAs start as its first chunks land), D tiles
  // ahead of their use; the last round computes what is left and loads
  // nothing.
  if constexpr (LDS) {
    // Staged form: step jt's 64 positions (wave w computes the 16 at 16 w)
    // land in LDS by direct-to-LDS loads, each 1 KiB piece from one wave,
    // while the previous step is computed. Row r's 16-byte K chunks are
    // stored XOR-permuted by r % 16 and V's (fp32) with bit 4 of the chunk
    // folded into bit 0, so the operand reads below are free of bank
    // conflicts; the operands and their clamping are the register form's.
    constexpr int kLPW = kStage / 1024 / W;  // pieces per wave per stage
    const int n_steps = (n_tiles + W - 1) / W;
    auto kq = [](int r, int q) { return q ^ (r & 15); };
    auto vq = [](int q) { return sizeof(T) == 4 ? q ^ ((q >> 4) & 1) : q; };
    auto stage = [&](int jt, int st) {
      jt = min(jt, n_steps - 1);  // past the last step: the last again (never read)
#pragma unroll
      for (int ii = 0; ii < kLPW; ++ii) {
        const int piece = wave + W * ii;
        const int o = piece * 1024 + 16 * lane, plane = o / kPlaneB, ob = o % kPlaneB;
        const int r = ob / kRowB, q = (ob % kRowB) / 16;
        const int t = min(t_begin + 64 * jt + r, t_end - 1);
        const T* src = (plane == 0 ? kl + (size_t)t * kv_dim + col + kq(r, q) * (16 / (int)sizeof(T))
                                   : vl + (size_t)t * kv_dim + col + vq(q) * (16 / (int)sizeof(T)));
        lds_load16(src, (lds_void*)(lds_raw + st * kStage + piece * 1024));
      }
    };
    auto read_tile = [&](int st, CT (&kb)[NKC], CT (&vb)[NVC]) {
      const char* base = lds_raw + st * kStage;
      const int rk = 16 * wave + li;
#pragma unroll
      for (int c = 0; c < NKC; ++c) kb[c] = *reinterpret_cast<const CT*>(base + rk * kRowB + kq(rk, lk + 4 * c) * 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rv = 16 * wave + 4 * lk + r;
#pragma unroll
        for (int h = 0; h < 8 / E; ++h)
          vb[r * (8 / E) + h] = *reinterpret_cast<const CT*>(base + kPlaneB + rv * kRowB +
                                                             vq((8 * li + E * h) * (int)sizeof(T) / 16) * 16);
      }
    };
    if (n_steps > 0) {
      stage(0, 0);
      scale_q();
      for (int jt = 0; jt < n_steps; ++jt) {
        wait_vmcnt<0>();  // this wave's pieces of step jt have landed
        __syncthreads();       // everyone's have, and step jt - 1's stage is free
        stage(jt + 1, (jt + 1) & 1);
        CT kb[NKC], vb[NVC];
        read_tile(jt & 1, kb, vb);
        if (wave + jt * W < n_tiles) compute(jt, kb, vb);
      }
      wait_vmcnt<0>();
    }
    __syncthreads();  // the ring's bytes become the merge's
  } else {
    CT kr[D][NKC], vr[D][NVC];
#pragma unroll
    for (int i = 0; i < D; ++i) load_tile(i, kr[i], vr[i]);
    __builtin_amdgcn_sched_barrier(0);
    scale_q();
    const int n_rounds = (my_tiles + D - 1) / D;
    for (int rr = 0; rr + 1 < n_rounds; ++rr) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        compute(rr * D + i, kr[i], vr[i]);
        load_tile((rr + 1) * D + i, kr[i], vr[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (n_rounds > 0) {
      const int j0 = (n_rounds - 1) * D;
#pragma unroll
      for (int i = 0; i < D; ++i)
        if (j0 + i < my_tiles) compute(j0 + i, kr[i], vr[i]);
    }
  }
  l_run = swap_sum<16>(l_run);
  l_run = swap_sum<32>(l_run);

  if constexpr (H16) {
#pragma unroll
    for (int b = 0; b < 8; ++b) o[b] *= 1.f / kPScale;  // the probabilities' scale, exactly
  }
  // o[b][r] = O^T[d = 8*(4*lk + r) + b][m = li]. Merge the W waves in LDS.
  auto sm_o = reinterpret_cast<float (*)[16][kD + 4]>(lds_raw);
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
  const __amdgpu_buffer_rsrc_t rs = ws_rsrc(mg.part, mg.ws_bytes);
  // XCD mode. Workgroups whose blockIdx agree mod 8 run on the same XCD (the
  // dispatcher deals workgroups to the 8 XCDs round robin; a probe at set-up
  // checks it), so the splits s of a kv head with s = r (mod 8) share an L2:
  // level-1 group r (its members' splits are r, r + 8, ...: fixed by n_splits
  // alone). A group of one writes its row straight to level 2.
  const int x_slot = split & 7;  // = (blockIdx.x - hidx * n_splits) mod 8
  const int x_n1 = (n_splits - 1 - x_slot) / 8 + 1;
  const uint32_t x_l2_row0 = (uint32_t)(gridDim.x + hidx * 8);
  const bool dev_rows = mg.mode == kMergeXcd && x_n1 == 1;
  const uint32_t my_row =
      mg.mode == kMergeXcd && x_n1 == 1 ? x_l2_row0 + (uint32_t)x_slot : (uint32_t)(hidx * n_splits + split);
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
      if (dev_rows) {  // device-scope stores for a hand-off across XCDs
        const uint32_t row = my_row * (uint32_t)stride * 4u;
        __builtin_amdgcn_raw_buffer_store_b128(O, rs, row + (uint32_t)(g * kD + d) * 4u, 0, kPolicyDevice);
        if (d == 0) {
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, M), rs,
                                                row + (uint32_t)(group * kD + 2 * g) * 4u, 0, kPolicyDevice);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, L), rs,
                                                row + (uint32_t)(group * kD + 2 * g + 1) * 4u, 0, kPolicyDevice);
        }
      } else {
        float* mine = mg.part + (size_t)my_row * stride;
        *reinterpret_cast<f32x4*>(mine + g * kD + d) = O;
        if (d == 0) {
          mine[group * kD + 2 * g] = M;
          mine[group * kD + 2 * g + 1] = L;
        }
      }
    }
  }
  if (n_splits == 1 || mg.mode == kMergeKernel) return;
  float* const head_out = out + (size_t)hidx * group * kD;

  // Level 1, inside this XCD: the last member to finish folds the group's
  // rows (plain stores, complete in this L2 before the ticket; loads that
  // skip the CU's L1 and hit this L2) in split order, and writes the group's
  // row to level 2 at device scope. Each counter has its own 128-byte line:
  // atomics on one line serialize.
  if (x_n1 > 1) {
    const int key = (int)(blockIdx.x & 7);  // the XCD slot this launch dealt the workgroup
    if (!last_of(mg.xt + (size_t)(key * mg.xpad + hidx) * 32, (unsigned)x_n1, tid)) return;
    fold_rows<NT, kPolicyL2>(rs, (uint32_t)(hidx * n_splits + x_slot), x_n1, stride, group,
                             x_l2_row0 + (uint32_t)x_slot, nullptr, tid, 8u);
  }
  // Level 2, across XCDs: the last group to finish folds the <= 8 group rows
  // in group order (device-scope rows and loads).
  const int n2 = min(8, n_splits);
  if (!last_of(mg.xt + (size_t)(8 * mg.xpad + hidx) * 32, (unsigned)n2, tid)) return;
  fold_rows<NT>(rs, x_l2_row0, n2, stride, group, 0, head_out, tid);
}

// fp32 log-sum-exp merge of the splits of every (kv head, subgroup of G
// heads) partial row set: one 256-thread workgroup per (query head of the
// range, block of 16 output columns). Thread t takes columns 4*(t % 4) .. +3
// of the block and the splits t/4, t/4 + 64, ...; it issues all of a round's
// loads (kMergePer splits, 16-byte o loads) before folding any, in split
// order, so up to 256 splits cost one memory round trip. Each wave's 16
// split lanes per column quad then fold by cross-lane exchange (lane i with
// lane i ^ 4, 8, 16, 32), and lane k of wave 0 folds the four waves through
// LDS in wave order: one barrier (a 6-level LDS tree with a barrier per
// level cost 0.12 µs more per call). The order is fixed by n_splits alone.
// Measured against one workgroup per query head (8 split lanes, 3-level
// tree) and one wave per 4 columns (a 64-lane butterfly), this spread was
// the fastest: the merge's bytes come from other XCDs' writes, and a CU's
// share of them bounds its time. 32 columns per workgroup (kMergeQuads 8:
// 512 threads, each partial's 128-byte line read by one workgroup instead
// of two) made the call 0.25 µs slower; non-temporal stores of the partials
// in the tile kernel, 0.18 µs slower.
constexpr int kMergeLanes = 64;
constexpr int kMergeQuads = 4;                   // column quads per workgroup (16 columns)
constexpr int kMergeBlock = 4 * kMergeQuads;     // output columns per workgroup
constexpr int kMergeThreads = 64 * kMergeQuads;  // 64 split lanes per column quad
template <int MP>  // splits per lane per round: 1, 2 or 4 (up to 64, 128, 256 splits in one round)
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(const float* __restrict__ part, int n_splits,
                                                                     int stride, int G, int group, int n_hg,
                                                                     float* __restrict__ out) {
  constexpr int kMergePer = MP;
  constexpr int QW = kMergeQuads;  // waves, and quads per lane group
  const int blk = blockIdx.x % (kD / kMergeBlock), h = blockIdx.x / (kD / kMergeBlock);  // h: q head in the range
  const int hidx = h / group, hh = h % group;
  const int g = hh % G, job = hidx * n_hg + hh / G;
  const int tid = threadIdx.x, k = tid % QW, sl = tid / QW;
  const int d = blk * kMergeBlock + 4 * k;
  const float* base = part + (size_t)job * n_splits * stride;
  float M = kNegSentinel, L = 0.f;
  f32x4 O = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n_splits; s0 += kMergeLanes * kMergePer) {
    f32x4 ov[kMergePer];
    float mv[kMergePer], lv[kMergePer];
#pragma unroll
    for (int i = 0; i < kMergePer; ++i) {
      const float* ps = base + (size_t)min(s0 + sl + i * kMergeLanes, n_splits - 1) * stride;
      ov[i] = *reinterpret_cast<const f32x4*>(ps + g * kD + d);
      mv[i] = ps[G * kD + 2 * g];
      lv[i] = ps[G * kD + 2 * g + 1];
    }
#pragma unroll
    for (int i = 0; i < kMergePer; ++i)
      if (s0 + sl + i * kMergeLanes < n_splits) {
        const float mn = fmaxf(M, mv[i]);
        const float a = __builtin_amdgcn_exp2f(M - mn), c = __builtin_amdgcn_exp2f(mv[i] - mn);
        L = L * a + lv[i] * c;
        O = O * a + ov[i] * c;
        M = mn;
      }
  }
  auto fold = [&](float m2, float l2, f32x4 o2) {
    const float mn = fmaxf(M, m2);
    const float a = __builtin_amdgcn_exp2f(M - mn), c = __builtin_amdgcn_exp2f(m2 - mn);
    L = L * a + l2 * c;
    O = O * a + o2 * c;
    M = mn;
  };
  // A wave's split lanes of each column quad fold by cross-lane exchange,
  // then lane k of wave 0 folds the waves in order.
#pragma unroll
  for (int off = QW; off < 64; off <<= 1) {
    f32x4 o2;
#pragma unroll
    for (int e = 0; e < 4; ++e) o2[e] = __shfl_xor(O[e], off, 64);
    fold(__shfl_xor(M, off, 64), __shfl_xor(L, off, 64), o2);
  }
  __shared__ float sm_m[QW][QW], sm_l[QW][QW];
  __shared__ f32x4 sm_o[QW][QW];
  const int wave = tid >> 6;
  if ((tid & 63) < QW) {
    sm_m[wave][k] = M;
    sm_l[wave][k] = L;
    sm_o[wave][k] = O;
  }
  __syncthreads();
  if (tid < QW) {
#pragma unroll
    for (int w = 1; w < QW; ++w) fold(sm_m[w][k], sm_l[w][k], sm_o[w][k]);
    const f32x4 r = O / L;  // out may be only 4-byte aligned
    float* op = out + (size_t)h * kD + d;
    op[0] = r[0];
    op[1] = r[1];
    op[2] = r[2];
    op[3] = r[3];
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
  const dim3 grid((unsigned)(n_q * (kD / kMergeBlock)));
  if (n_splits <= kMergeLanes)
    hipLaunchKernelGGL(decode_merge_kernel<1>, grid, dim3(kMergeThreads), 0, s, part, n_splits, part_stride_of(G), G, group,
                       n_hg, out);
  else if (n_splits <= 2 * kMergeLanes)
    hipLaunchKernelGGL(decode_merge_kernel<2>, grid, dim3(kMergeThreads), 0, s, part, n_splits, part_stride_of(G), G, group,
                       n_hg, out);
  else
    hipLaunchKernelGGL(decode_merge_kernel<4>, grid, dim3(kMergeThreads), 0, s, part, n_splits, part_stride_of(G), G, group,
                       n_hg, out);
}

// Launch shape of the MFMA tile kernel. Default, from sweeps on MI355X:
// 4-wave workgroups; splits of one 64-position step (one 16-position tile
// per wave) while that keeps at most one workgroup per CU (4 kv heads: up
// to 4096 positions), then an even share of the positions in 16-position
// steps on one workgroup per CU up to 448 positions each, then on two (so
// about kTileWaves waves, two per SIMD, all resident at once: 128 splits
// of 256 positions per kv head at 32768). Between the powers of two this
// runs 7-14 % faster than whole steps with two workgroups per CU past 128
// positions (fp32: 4097 positions 9.7 vs 11.1 µs, 6000 10.4 vs 12.0,
// 12000 14.6 vs 16.1; f16: 12000 11.2 vs 12.5, 20000 13.9 vs 15.0), which
// leave a few CUs running two workgroups. Each wave takes its
// share of the split's tiles one at a time (ring depth 1: the next tile's
// loads issue once the current one is computed): two or four of a wave's
// tiles in flight measured 0-6 % slower (config 5, f16 at 32768: 19.6 vs
// 18.6 µs; fp32 at 16384: 19.1 vs 17.9 µs), since the SIMD's other
// resident wave covers a wave's load latency. A pinned split that leaves
// fewer waves keeps a slot per tile. The splits of a kv head
// are folded by decode_merge_kernel, or by the XCD merge (merge_mode). The
// split length is sized for the cache's kv heads and every other field
// derives from it and positions, so a kv-head range takes the same
// reduction tree as the whole call.
constexpr int kTileWaves = 2048;
struct TilePlan {
  int waves, depth, split_len, n_splits;
  int merge;  // MergeMode
  bool lds;  // RV_TUNE_DECODE_IMPL 3: tiles staged through LDS (4 waves, depth 1)
};

// Ring depth: one tile at a time for the default plan, or when the whole
// cache's grid (every kv head, so a kv-head range picks the same depth)
// holds about kTileWaves waves; for a pinned long split with fewer waves, a
// slot per tile of the wave's share up to the ring's limit, since no other
// wave covers the loads.
static int tile_depth(const rv_kv* kv, int waves, int split_len, int n_splits) {
  const int tpw = (split_len / 16 + waves - 1) / waves;  // tiles per wave
  const long grid_waves = (long)n_splits * (long)kv->n_kv_heads * waves;
  const bool one = kv->tune_decode_split_len <= 0 || grid_waves >= kTileWaves;  // the default plan, or a full grid
  int d = kv->tune_decode_depth > 0 ? (int)kv->tune_decode_depth : one ? 1 : tpw;
  const int dmax = kv->elem == RV_ELEM_F32 ? 2 : 4;  // register ring: 64 (f32) or 32 (f16) VGPRs per tile
  d = std::min(d, dmax);
  return d >= 4 ? 4 : d >= 2 ? 2 : 1;
}

// RV_TUNE_DECODE_MERGE: 0 auto, 1 the in-launch XCD merge, 2 the separate
// merge kernel. The XCD merge needs the dispatcher's round-robin dealing,
// which rv_kv_new checks on the cache's device (kv->xcd_ok); without it every
// choice is the separate kernel. Auto takes the XCD merge up to kXcdAuto
// splits per kv head, where each split is its own level-1 group and only the
// hand-off across XCDs remains (48-layer graphs, µs per call, separate kernel
// vs XCD merge: f32 129 positions (3 splits) 7.65 vs 6.85, 257 7.84 vs 7.06,
// 512 7.86 vs 7.19; f16 193 6.36 vs 5.54, 512 6.60 vs 5.88). Past 8 splits
// the first level adds a second ticket round trip and the XCD merge loses
// (f32 513: 7.95 vs 8.43, 4096: 8.90 vs 9.42; f16 32768: 18.1 vs 19.4).
constexpr int kXcdAuto = 8;
static int merge_mode(const rv_kv* kv, int n_splits) {
  if (!kv->xcd_ok) return kMergeKernel;
  switch (kv->tune_decode_merge) {
    case 1: return kMergeXcd;
    case 2: return kMergeKernel;
    default: return n_splits <= kXcdAuto ? kMergeXcd : kMergeKernel;
  }
}

static TilePlan plan_tile(const rv_kv* kv, long positions) {
  TilePlan p;
  const int64_t tw = kv->tune_decode_waves;
  p.waves = tw == 8 ? 8 : tw == 2 ? 2 : tw == 1 ? 1 : 4;
  const int step = p.waves * 16;
  long len = kv->tune_decode_split_len;
  bool fine = false;  // a default length in 16-position steps
  if (len <= 0 && positions * (long)kv->n_kv_heads > (long)kCUs * step) {
    // Past one step per workgroup on one workgroup per CU, whole steps would
    // leave a few CUs running two workgroups (4097 positions: 65 splits x 4
    // kv heads = 260 workgroups, 11.1 vs 9.7 us per call). The split instead
    // takes an even share of the positions in 16-position steps: one
    // workgroup per CU up to 7 steps (448 positions) each, then two (at
    // 32768 positions that is 256 each, 18.4 vs 18.7 us for one workgroup
    // of 512; at 28000 one workgroup of 448 takes 16.5 vs 17.2 us). Sized
    // for the whole cache's kv heads, so a kv-head range takes the whole
    // call's splits.
    const long share = positions * (long)kv->n_kv_heads;
    long per = (share + kCUs - 1) / kCUs;
    if (per > 7 * step) per = (share + 2 * kCUs - 1) / (2 * kCUs);
    len = std::max<long>((per + 15) / 16 * 16, step);
    fine = true;
  } else if (len <= 0 && positions <= 3L * step &&
             positions * 2 * (long)kv->head_dim * (kv->elem == RV_ELEM_F32 ? 4 : 2) <= (128L << 10)) {
    // At most 3 tiles per wave and 128 KiB of K and V per kv head: one split
    // per kv head, its waves taking the tiles one at a time, and no merge
    // launch. Graph-replayed calls, one layer (cache-resident) / 48 layers,
    // against 64-position splits: f16 128 positions 4.1 / 4.2 vs 6.1 / 6.2
    // us, 192 4.6 / 5.6 vs 6.2 / 6.3; fp32 128 6.0 / 6.9 vs 7.3 / 7.5. Each
    // further tile per wave is another memory round trip: f16 256 (4 per
    // wave) 5.2 / 6.9 vs 6.2 / 6.3, fp32 256 8.3 vs 7.3.
    len = positions;
  } else if (len <= 0) {
    len = step;  // one step per workgroup, at most one workgroup per CU
  }
  len = std::max<long>(len, step);
  p.split_len = fine ? (int)len : (int)((len + step - 1) / step * step);
  p.n_splits = (int)((positions + p.split_len - 1) / p.split_len);
  p.depth = tile_depth(kv, p.waves, p.split_len, p.n_splits);
  p.lds = kv->tune_decode_impl == 3 && p.waves == 4;
  if (p.lds) p.depth = 1;
  p.merge = merge_mode(kv, p.n_splits);
  return p;
}

// Workspace floats of a plan: level-1 rows, then level-2 rows.
static size_t tile_ws_floats(const TilePlan& p, int n_heads, int group) {
  const size_t rows = (size_t)n_heads * (p.n_splits + (p.merge == kMergeXcd ? 8 : 0));
  return rows * part_stride_of(group);
}

// The largest workspace any tile plan of this cache can ask for at up to
// `capacity` positions: the default length keeps n_splits * n_heads at most
// about kTileWaves / 4 + n_heads (split_len >= 64 * tiles-per-wave), a pinned
// length gives capacity / split_len splits; n_grp <= n_splits.
static size_t tile_ws_bound(const rv_kv* kv, int n_heads, int group) {
  const long cap = (long)kv->capacity;
  long splits = (cap + 63) / 64;
  if (kv->tune_decode_split_len > 0)
    splits = (cap + kv->tune_decode_split_len - 1) / kv->tune_decode_split_len;
  else
    splits = std::min<long>(splits, kTileWaves / 4 / n_heads + 2);
  splits = std::max<long>(splits, 1);
  return (size_t)n_heads * (2 * (size_t)splits + 8) * part_stride_of(group);
}

template <typename T, int W, int D, bool PRO, bool H16, typename Pro>
static void launch_tile_wd(const TimedPair& tp, dim3 grid, hipStream_t s, const float* q, const void* kl,
                           const void* vl, int kv_dim, int positions, int split_len, int n_splits, int group,
                           int kv_lo, float qscale, const MergeArgs& mg, float* out, const Pro& pro) {
  launch_timed(tp, decode_tile_kernel<T, W, D, PRO, H16>, grid, dim3(W * 64), s, q, (PlanePtr<PRO, T>)kl,
               (PlanePtr<PRO, T>)vl, kv_dim, positions, split_len, n_splits, group, kv_lo, qscale, mg, out, pro);
}

template <typename T, bool PRO, bool H16, typename Pro>
static void launch_tile(const TilePlan& p, const TimedPair& tp, hipStream_t s, int n_heads, const float* q,
                        const void* kl, const void* vl, int kv_dim, int positions, int group, int kv_lo, float qscale,
                        const MergeArgs& mg, float* out, const Pro& pro) {
  const dim3 grid((unsigned)(n_heads * p.n_splits));
  if constexpr (!PRO) {
    if (p.lds) {
      launch_timed(tp, decode_tile_kernel<T, 4, 1, false, H16, true>, grid, dim3(256), s, q, (PlanePtr<false, T>)kl,
                   (PlanePtr<false, T>)vl, kv_dim, positions, p.split_len, p.n_splits, group, kv_lo, qscale, mg, out,
                   pro);
      return;
    }
  }
#define RV_TILE(W, D)                                                                                              \
  launch_tile_wd<T, W, D, PRO, H16>(tp, grid, s, q, kl, vl, kv_dim, positions, p.split_len, p.n_splits, group, kv_lo, \
                                    qscale, mg, out, pro)
  // Depth 4 only for f16 planes (fp32 tiles would spill).
  constexpr int D4 = std::is_same<T, float>::value ? 2 : 4;
  if (p.waves == 8) {
    if (p.depth == 1) RV_TILE(8, 1);
    else if (p.depth == 2) RV_TILE(8, 2);
    else RV_TILE(8, D4);
  } else if (p.waves == 2) {
    if (p.depth == 1) RV_TILE(2, 1);
    else if (p.depth == 2) RV_TILE(2, 2);
    else RV_TILE(2, D4);
  } else if (p.waves == 1) {
    if (p.depth == 1) RV_TILE(1, 1);
    else if (p.depth == 2) RV_TILE(1, 2);
    else RV_TILE(1, D4);
  } else {
    if (p.depth == 1) RV_TILE(4, 1);
    else if (p.depth == 2) RV_TILE(4, 2);
    else RV_TILE(4, D4);
  }
#undef RV_TILE
}

// Workspace and merge arguments of a tile plan; grows the workspace (sized
// for the cache's capacity) on first need.
static HipStatus tile_merge_args(rv_kv* kv, const TilePlan& p, int n_heads, int group, const Workspace* ws,
                                 MergeArgs* mg) {
  const size_t need = tile_ws_floats(p, n_heads, group) * sizeof(float);
  HipStatus st;
  if (ws) {
    if (need > ws->bytes) {
      st.e = hipErrorInvalidValue;
      st.what = "decode scratch too small";
      return st;
    }
    mg->part = (float*)ws->base;
    mg->ws_bytes = (uint32_t)std::min<size_t>(ws->bytes, 0xFFFFFFF0u);
  } else {
    st = ensure_workspace(kv, need, tile_ws_bound(kv, n_heads, group) * sizeof(float));
    if (st.e != hipSuccess) return st;
    mg->part = (float*)kv->ws;
    mg->ws_bytes = (uint32_t)std::min<size_t>(kv->ws_bytes, 0xFFFFFFF0u);
  }
  mg->xt = xcd_tickets(kv);
  mg->xpad = (int)xcd_ticket_pad(kv);
  mg->mode = p.merge;
  return st;
}

size_t decode_ws_bound(const rv_kv* kv) {
  if (kv->head_dim != kD) return 0;
  return tile_ws_bound(kv, (int)kv->n_kv_heads, 16) * sizeof(float);
}

bool decode_pro_supported(const rv_kv* kv, size_t n_q_heads) {
  return kv->head_dim == kD && n_q_heads % kv->n_kv_heads == 0 && n_q_heads / kv->n_kv_heads <= 16 &&
         kv->tune_decode_impl != 1;
}

namespace {
// A token graph's last node: the next token's position (one lane's store).
__global__ __launch_bounds__(64) void position_advance_kernel(uint32_t* __restrict__ p, uint32_t n) {
  if (threadIdx.x == 0) p[0] += n;
}
}  // namespace

HipStatus launch_position_advance(uint32_t* d_position, uint32_t n, hipStream_t s) {
  HipStatus st;
  hipLaunchKernelGGL(position_advance_kernel, dim3(1), dim3(64), 0, s, d_position, n);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "position advance launch";
  return st;
}

HipStatus launch_decode_pro(rv_kv* kv, const float* q_raw, size_t n_q_heads, size_t layer, size_t positions,
                            float scale, const DecodePro& pro, float* out, hipStream_t s) {
  const int n_heads = (int)kv->n_kv_heads;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const TilePlan p = plan_tile(kv, (long)positions);
  MergeArgs mg;
  HipStatus st = tile_merge_args(kv, p, n_heads, group, nullptr, &mg);
  if (st.e != hipSuccess) return st;
  const TimedPair tp = timing_pair(kv, s);
  const float qscale = scale * kLog2e;
  const void* kl = kv->k_layer(layer);
  const void* vl = kv->v_layer(layer);
  if (kv->elem == RV_ELEM_F32)
    launch_tile<float, true, false>(p, tp, s, n_heads, q_raw, kl, vl, (int)kv->kv_dim, (int)positions, group, 0,
                                    qscale, mg, out, pro);
  else
    launch_tile<_Float16, true, false>(p, tp, s, n_heads, q_raw, kl, vl, (int)kv->kv_dim, (int)positions, group, 0,
                                       qscale, mg, out, pro);
  if (p.n_splits > 1 && p.merge == kMergeKernel)
    launch_merge(mg.part, p.n_splits, group, group, 1, n_heads * group, out, s);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "decode launch";
  return st;
}

size_t decode_ws_need(const rv_kv* kv, size_t n_q_heads, size_t positions, size_t n_heads) {
  if (n_heads == 0) return 0;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  if (kv->head_dim == kD && group <= 16 && kv->tune_decode_impl != 1)
    return tile_ws_floats(plan_tile(kv, (long)positions), (int)n_heads, group) * sizeof(float);
  if (kv->head_dim == kD) {
    const DecodeShape d = pick_shape(kv, (int)positions, (int)n_heads, group);
    const size_t n_splits = (positions + d.split_len - 1) / d.split_len;
    return n_heads * (size_t)(group / d.hg_size) * n_splits * part_stride_of(d.hg_size) * sizeof(float);
  }
  return n_heads * (size_t)group * positions * sizeof(float);
}

HipStatus launch_decode(rv_kv* kv, const float* q, size_t n_q_heads, size_t layer, size_t positions,
                        float scale, size_t kv_lo, size_t kv_hi, float* out, hipStream_t s, const Workspace* ws) {
  HipStatus st;
  if (ws && decode_ws_need(kv, n_q_heads, positions, kv_hi - kv_lo) > ws->bytes) {
    st.e = hipErrorInvalidValue;
    st.what = "decode scratch too small";
    return st;
  }
  // With a caller's workspace nothing may allocate: no timing events either.
  auto timing = [&]() { return ws ? TimedPair{} : timing_pair(kv, s); };
  const int n_heads = (int)(kv_hi - kv_lo);
  if (n_heads == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const void* kl = kv->k_layer(layer);
  const void* vl = kv->v_layer(layer);
  const float qscale = scale * kLog2e;
  if (kv->head_dim == kD && group <= 16 && kv->tune_decode_impl != 1) {
    const TilePlan p = plan_tile(kv, (long)positions);
    MergeArgs mg;
    st = tile_merge_args(kv, p, n_heads, group, ws, &mg);
    if (st.e != hipSuccess) return st;
    const TimedPair tp = timing();
    const int kvd = (int)kv->kv_dim;
    if (kv->elem == RV_ELEM_F32)
      launch_tile<float, false, false>(p, tp, s, n_heads, q, kl, vl, kvd, (int)positions, group, (int)kv_lo, qscale,
                                       mg, out, NoPro{});
    else if (kv->tune_decode_impl == 2)  // fp32 MFMA operands for f16 planes (the reference form)
      launch_tile<_Float16, false, false>(p, tp, s, n_heads, q, kl, vl, kvd, (int)positions, group, (int)kv_lo,
                                          qscale, mg, out, NoPro{});
    else
      launch_tile<_Float16, false, true>(p, tp, s, n_heads, q, kl, vl, kvd, (int)positions, group, (int)kv_lo, qscale,
                                         mg, out, NoPro{});
    if (p.n_splits > 1 && p.merge == kMergeKernel)
      launch_merge(mg.part, p.n_splits, group, group, 1, n_heads * group, out, s);
  } else if (kv->head_dim == kD) {
    const DecodeShape d = pick_shape(kv, (int)positions, n_heads, group);
    const int n_hg = group / d.hg_size;
    const int n_splits = (int)((positions + d.split_len - 1) / d.split_len);
    const int n_jobs = n_heads * n_hg;
    const size_t part_bytes = (size_t)n_jobs * n_splits * part_stride_of(d.hg_size) * sizeof(float);
    float* part = ws ? (float*)ws->base : nullptr;
    if (!ws) {
      const size_t bound_splits = std::max<size_t>(1, (kv->capacity + 15) / 16);
      st = ensure_workspace(kv, part_bytes,
                            (size_t)n_jobs * bound_splits * part_stride_of(d.hg_size) * sizeof(float));
      if (st.e != hipSuccess) return st;
      part = (float*)kv->ws;
    }
    SplitArgs a{q, kl, vl, (int)kv->kv_dim, (int)positions, d.split_len, n_splits, n_heads * n_splits, group,
                n_hg, (int)kv_lo, qscale, part, out, timing()};
    if (kv->elem == RV_ELEM_F32) {
      if (d.waves == 4) launch_split_g<float, 4>(d.hg_size, a, s);
      else launch_split_g<float, 8>(d.hg_size, a, s);
    } else {
      if (d.waves == 4) launch_split_g<_Float16, 4>(d.hg_size, a, s);
      else launch_split_g<_Float16, 8>(d.hg_size, a, s);
    }
    if (n_splits > 1) launch_merge(part, n_splits, d.hg_size, group, n_hg, n_jobs * d.hg_size, out, s);
  } else {
    const size_t hd = kv->head_dim;
    const int n_qr = n_heads * group;
    float* scores = ws ? (float*)ws->base : nullptr;
    if (!ws) {
      st = ensure_workspace(kv, (size_t)n_qr * positions * sizeof(float),
                            (size_t)n_qr * kv->capacity * sizeof(float));
      if (st.e != hipSuccess) return st;
      scores = (float*)kv->ws;
    }
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

// ---- the dispatcher's XCD dealing ---------------------------------------------------
namespace {
// Each workgroup records the XCD it runs on (the XCC_ID hardware register).
__global__ __launch_bounds__(64) void xcd_probe_kernel(uint32_t* __restrict__ out) {
  if (threadIdx.x == 0) out[blockIdx.x] = __builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xf;  // HW_REG_XCC_ID
}
constexpr int kProbeBlocks = 1024;
std::mutex g_xcd_mu;
int g_xcd_state[64] = {};  // per device: 0 unknown, 1 ok, 2 not
}  // namespace

// Whether, on `device` (current), the workgroups of a launch whose indices
// agree mod 8 run on one XCD: four probe launches of 1024 workgroups, every
// workgroup's XCC_ID compared with that of workgroup b mod 8, and the 8 slots
// on 8 distinct XCDs. Cached per device.
bool xcd_dealing_ok(int device) {
  if (device < 0 || device >= 64) return false;
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  if (g_xcd_state[device]) return g_xcd_state[device] == 1;
  bool ok = true;
  uint32_t* d = nullptr;
  std::vector<uint32_t> h(kProbeBlocks);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess || prop.multiProcessorCount != (int)kCUs ||
      hipMalloc(&d, kProbeBlocks * sizeof(uint32_t)) != hipSuccess)
    ok = false;
  for (int rep = 0; ok && rep < 4; ++rep) {
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(kProbeBlocks), dim3(64), 0, nullptr, d);
    if (hipMemcpy(h.data(), d, kProbeBlocks * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) {
      ok = false;
      break;
    }
    unsigned seen = 0;
    for (int b = 0; b < 8; ++b) seen |= 1u << h[b];
    ok = seen == 0xffu;
    for (int b = 8; ok && b < kProbeBlocks; ++b) ok = h[b] == h[b % 8];
  }
  if (d) (void)hipFree(d);
  (void)hipGetLastError();
  g_xcd_state[device] = ok ? 1 : 2;
  return ok;
}

// ---- the no-alloc entry point's scratch ------------------------------------------
// rv_decode_attention_noalloc's split partials (or scores, on the generic
// path) live here instead of in the cache's workspace: a fixed array that
// each GPU the library runs on holds until the process ends. In host code
// the name is only a stand-in; the array's device address, one per device,
// comes from hipGetSymbolAddress with that device current, and only that
// address reaches kernels. Nothing in it must start at zero (every partial
// is written before it is read). Calls that overlap on one GPU share it and
// race.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

HipStatus noalloc_scratch(int device, void** ptr) {
  HipStatus st;
  *ptr = nullptr;
  if (device < 0 || device >= kMaxScratchDevices) {
    st.e = hipErrorInvalidDevice;
    st.what = "device index for the no-alloc scratch";
    return st;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    st.e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st.e != hipSuccess) {
      st.what = "hipGetSymbolAddress(scratch)";
      return st;
    }
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return st;
}

}  // namespace rv
