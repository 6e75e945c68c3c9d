// rv_prologue.hip — per-head QK-RMSNorm + NeoX RoPE and the KV append.
//
// Replaces, per token row, rmsnorm_in_place over each head
// (crates/core/src/kernels/primitives/norm.rs:18-26, :72-90), rope_neox_heads
// (primitives/rope.rs:31-45, :82-105) and KvCache::append (kv/mod.rs:336-368),
// as called at model/forward.rs:2622-2631 and model/prefill.rs:2057-2087.
//
// One wavefront per 4 heads of a row (q, k and v heads in one launch). The
// f32 arithmetic is the reference's, op for op and with contraction off: `x * inv * w` left to right, the rotation
// as two separately rounded products and a subtraction/addition. The mean of
// squares is summed in f64 (a tree, not the reference's sequential order: the
// two agree to f64 rounding before the cast to f32). RoPE angles are
// `pos * inv_freq` in f64 with inv_freq computed on the host in f64, then
// sin/cos in f64 and cast to f32, as rope.rs:35-39 does.
#include "rv_device.hpp"
#include "rv_internal.hpp"
#include "rv_staged.hpp"

#include <math.h>

namespace rv {

void fill_inv_freq(InvFreq& t, size_t head_dim, float theta) {
  const double base = (double)theta;
  const double dim = (double)head_dim;
  for (size_t i = 0; i < head_dim / 2 && i < (size_t)kMaxHalf; ++i) t.f[i] = pow(base, -2.0 * (double)i / dim);
}

namespace {

template <typename T>
__device__ __forceinline__ void store_elem(T* p, float v);
template <>
__device__ __forceinline__ void store_elem<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_elem<uint16_t>(uint16_t* p, float v) {
  *p = f32_to_f16_bits(v);
}

// Stores v as the cache's element type; returns what the cache now holds,
// as f32 (what the prefill stage kernel would read back).
template <typename T>
__device__ __forceinline__ float store_cached(T* p, float v);
template <>
__device__ __forceinline__ float store_cached<float>(float* p, float v) {
  *p = v;
  return v;
}
template <>
__device__ __forceinline__ float store_cached<uint16_t>(uint16_t* p, float v) {
  const uint16_t b = f32_to_f16_bits(v);
  *p = b;
  return (float)__builtin_bit_cast(_Float16, b);
}

// The staged tiles a prefill chunk's prologue writes its k and v rows into
// (positions row0 + r; rows [rows, grid rows) are the rest of the last tile).
struct StagedRows {
  char* base;
  int tile_stride;
  int rows;
  long row0;
};

// Element d of kv head h's K (kind 0) or V (kind 1) row at position p, in
// the staged layout of mode SM: hi, and lo in the split mode.
template <int SM>
__device__ __forceinline__ void stage_elem(const StagedRows& sr, int kind, int h, long p, int d, float x) {
  typedef typename Op<SM>::E E;
  constexpr int P = kPlanes<SM>;
  const int t = (int)(p % kBT);
  char* tile = sr.base + ((size_t)h * sr.tile_stride + (size_t)(p / kBT)) * (2 * P * kPlaneBytes);
  char* dst = kind == 0 ? tile + k_off(t, d >> 3) + 2 * (d & 7) : tile + P * kPlaneBytes + vt_byte_m<SM>(d, t);
  const E hi = (E)x;
  *reinterpret_cast<E*>(dst) = hi;
  if constexpr (Op<SM>::kSplit) *reinterpret_cast<E*>(dst + kPlaneBytes) = (E)(x - (float)hi);
}

// A staging prologue's V rows, four positions [p0, p0 + 4) of kv head h per
// wave (p0 a multiple of 4 counted from row0's quad): the chunk's rows are
// copied into the cache, and each lane's two V^T elements (dims lane and
// lane + 64) of the four positions, which share one 8-byte piece of a V^T
// chunk, are written with one store per plane. Positions past the chunk in
// its last tile are staged as zeros; positions before row0 (already staged)
// are left alone, so a quad holding some takes 2-byte stores.
template <typename T, int SM>
__device__ __forceinline__ void stage_v_quad(const float* __restrict__ v, T* __restrict__ vp, int n_kv, int h,
                                             const StagedRows& sr, int g, int lane) {
  typedef typename Op<SM>::E E;
  typedef typename Op<SM>::V4 V4;
  constexpr int P = kPlanes<SM>;
  const long p0 = (sr.row0 & ~3L) + 4L * g;
  const long tile_end = (sr.row0 + sr.rows + kBT - 1) / kBT * kBT;
  if (p0 >= tile_end) return;
  float x[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long r = p0 + i - sr.row0;
    const bool live = r >= 0 && r < sr.rows;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const size_t at = ((size_t)(live ? r : 0) * n_kv + h) * 128 + lane + 64 * k;
      x[i][k] = live ? v[at] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long r = p0 + i - sr.row0;
    if (r < 0 || r >= sr.rows) continue;
#pragma unroll
    for (int k = 0; k < 2; ++k) x[i][k] = store_cached<T>(vp + ((size_t)r * n_kv + h) * 128 + lane + 64 * k, x[i][k]);
  }
  char* plane = sr.base + ((size_t)h * sr.tile_stride + (size_t)(p0 / kBT)) * (2 * P * kPlaneBytes) + P * kPlaneBytes;
  const int t = (int)(p0 % kBT);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    char* dst = plane + vt_byte_m<SM>(lane + 64 * k, t);  // positions t .. t + 3: 8 contiguous bytes
    V4 hi, lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hi[i] = (E)x[i][k];
      lo[i] = (E)(x[i][k] - (float)hi[i]);
    }
    if (p0 >= sr.row0) {
      *reinterpret_cast<V4*>(dst) = hi;
      if constexpr (P == 2) *reinterpret_cast<V4*>(dst + kPlaneBytes) = lo;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (p0 + i < sr.row0) continue;
        *reinterpret_cast<E*>(dst + 2 * i) = hi[i];
        if constexpr (P == 2) *reinterpret_cast<E*>(dst + kPlaneBytes + 2 * i) = lo[i];
      }
    }
  }
}

// grid (rows, n_kv_heads), one wave each: K and V heads copied into the
// cache, converted to the plane's element type (KvCache::append as is).
template <typename T>
__global__ __launch_bounds__(64) void append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                    T* __restrict__ kp, T* __restrict__ vp, int kv_dim, int hd) {
  const size_t src = (size_t)blockIdx.x * kv_dim + (size_t)blockIdx.y * hd;
  for (int i = threadIdx.x; i < hd; i += 64) {
    store_elem<T>(kp + src + i, k[src + i]);
    store_elem<T>(vp + src + i, v[src + i]);
  }
}

// One workgroup of a staging launch's query preparation: the 32 columns
// [32 wv, 32 wv + 32) of unit u (qw = u * VG + wv) in the prepared layout,
// wave wib taking columns 8 wib .. 8 wib + 7. Loads are whole vectors: load
// k brings column 8 wib + 2 k + (lane / 32) with lane l holding d = 4 (l %
// 32) .. + 3, so each load is 1 KiB contiguous (two columns' 512 bytes of
// q; a row's (cos, sin) pair halves), and the rope pair (d, d + 64) sits in
// lanes 16 apart (exchanged with one permlane16 swap). RMSNorm sums the
// column's squares in f64 over its 32 lanes (DPP within 16-lane rows, then
// the swap), then `x * inv * w` and the rotation in the reference's
// separately rounded f32 operations, times log2(e) * scale, rounded to the
// MFMA type. The columns turn around through the workgroup's 8 KiB of LDS
// (lq: column c's 16-byte chunk k at byte 256 c + 16 (k ^ (c & 15))), and
// wave wib stores operand blocks 2 wib and 2 wib + 1 whole. Columns past the
// chunk's rows are zeros. Every wave of the workgroup calls it (a barrier).
template <int SM>
__device__ __forceinline__ void prep_q_block(int qw, bool live, const float* __restrict__ q, int n_q,
                                             const float* __restrict__ q_w, float eps, long pos0, int rows,
                                             const QPrep& qp, int wib, int lane, uint16_t* lq) {
#pragma clang fp contract(off)
  typedef typename Op<SM>::E E;
  typedef typename Op<SM>::V8 V8;
  typedef E E4 __attribute__((ext_vector_type(4)));
  const int VG = qp.vectors / 32;
  const int u = qw / VG, wv = qw % VG;
  const int kvh = u / qp.n_rb, rb = u % qp.n_rb;
  const int hl = lane >> 5, dl = lane & 31;  // column parity of a load, d = 4 dl .. 4 dl + 3
  const bool first = dl < 16;                // d < 64: the first element of its rope pair
  if (live) {
    const f32x4 w_own = *reinterpret_cast<const f32x4*>(q_w + 4 * dl);
    f32x4 x[4], t[4];
    bool ok[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = 8 * wib + 2 * k + hl, m = 32 * wv + c;
      const int row = rb * qp.qr + m % qp.qr;
      ok[k] = row < rows;
      const int q_row = ok[k] ? row : rb * qp.qr;  // a row of the unit (its first is in the chunk)
      x[k] = *reinterpret_cast<const f32x4*>(q + ((size_t)q_row * n_q + (size_t)(kvh * qp.group + m / qp.qr)) * 128 +
                                             4 * dl);
      // cos of pairs 4 dl .. + 3 in the first lanes, sin in their partners
      t[k] = *reinterpret_cast<const f32x4*>(qp.rope + (size_t)(pos0 + q_row) * 128 + 4 * dl);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (!ok[k]) x[k] = f32x4{};
      double ss = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += (double)x[k][e] * (double)x[k][e];
      ss += dpp_f64<DPP_QUAD_XOR1>(ss);
      ss += dpp_f64<DPP_QUAD_XOR2>(ss);
      ss += dpp_f64<DPP_ROW_HALF_MIRROR>(ss);
      ss += dpp_f64<DPP_ROW_MIRROR>(ss);
      ss = swap_sum_f64<16>(ss);  // the column's 32 lanes
      const float inv = (float)(1.0 / sqrt(ss / 128.0 + (double)eps));
      f32x4 a, ap, tp, y;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = x[k][e] * inv * w_own[e];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const auto ra = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[e]), __float_as_uint(a[e]), false, false);
        const auto rt = __builtin_amdgcn_permlane16_swap(__float_as_uint(t[k][e]), __float_as_uint(t[k][e]), false,
                                                         false);
        ap[e] = __uint_as_float(first ? ra[1] : ra[0]);
        tp[e] = __uint_as_float(first ? rt[1] : rt[0]);
      }
      // first lanes: y = a0 cos - a1 sin; partners: y = a0 sin + a1 cos.
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float cs = first ? t[k][e] : tp[e], sn = first ? tp[e] : t[k][e];
        y[e] = first ? a[e] * cs - ap[e] * sn : ap[e] * sn + a[e] * cs;
      }
      E4 h;
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = (E)(y[e] * qp.qscale);
      const int c = 8 * wib + 2 * k + hl, d = 4 * dl;
      *reinterpret_cast<E4*>(lq + 128 * c + 8 * ((d >> 3) ^ (c & 15)) + (d & 7)) = h;
    }
  }
  __syncthreads();
  if (!live) return;
  const int lc = lane & 31, g = lane >> 5;
  // Non-temporal stores: the attention launch reads the operands, and this
  // launch's end has fewer dirty lines to write back (config 3 call 19.25 ->
  // 18.9 us).
  V8* dst = reinterpret_cast<V8*>(qp.base) + (size_t)qw * 8 * 64 + lane;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ks = 2 * wib + i;
    __builtin_nontemporal_store(*reinterpret_cast<const V8*>(lq + 128 * lc + 8 * ((2 * ks + g) ^ (lc & 15))),
                                dst + 64 * ks);
  }
}

// One decode or prefill row's prologue: q heads RMSNormed + rotated into
// q_out, k heads RMSNormed + rotated into the cache, v heads copied into the
// cache. grid (rows, slot blocks), one wave per 4 head slots of the row's
// list [q heads | k heads | v heads]. Lane l owns the element pairs
// (i, i + half) with i = l + 64 j, j < NP, for every head of its slots, so
// the row's sin/cos (f64, cast to f32) are computed once per wave rather than
// once per head, while the wave's head loads are in flight.
// SM >= 0 (a prefill chunk, head_dim 128): k and v rows, as the cache holds
// them, are also written into the staged tiles in mode SM, and the rest of
// the chunk's last tile is zeroed. The slot list is then the q heads (none,
// or into the prepared layout qp, rounded to SM's type) and the k heads, one
// per wave (grid rows past the chunk zero their K rows); v heads are handled by the
// blocks y >= the q and k slot blocks, one per (quad of positions x, head y
// - those blocks): stage_v_quad.
constexpr int kSlots = 4;
// Waves per block of a staging launch (the slot blocks of one row side by
// side: a prefill chunk's q, k and v heads are 8 + 1 + 4 blocks of a row at
// GQA 32/4, each short, so blocks of one wave spend more on dispatch than on
// work); other launches use one-wave blocks.
constexpr int kPrologueWaves = 4;

template <typename T, int NP, int SM>
__global__ __launch_bounds__(kPrologueWaves * 64) void row_prologue_kernel(const float* __restrict__ q, float* __restrict__ q_out,
                                                          int n_q, const float* __restrict__ k,
                                                          const float* __restrict__ v, T* __restrict__ kp,
                                                          T* __restrict__ vp, int n_kv, int hd,
                                                          const float* __restrict__ q_w,
                                                          const float* __restrict__ k_w, float eps, InvFreq inv,
                                                          long pos0, float* __restrict__ tab, StagedRows sr,
                                                          QPrep qp) {
#pragma clang fp contract(off)
  // Slots per wave: a staging launch gives each k head a wave of its own
  // (its f64 norm is a dependent chain of ~100 instructions; four of them
  // in one wave took 2.1-2.6 us after the loads landed), the others four.
  constexpr int KS = SM >= 0 ? 1 : kSlots;
  const int r = blockIdx.x, lane = threadIdx.x & 63;
  const int half = hd / 2;
  // This wave's slot block: blockIdx.y in one-wave blocks, the block's
  // waves side by side in a staging launch's (each wave independent; only
  // the query-preparation workgroups below share a barrier, all four of
  // their waves taking it).
  const int wib = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // With prepared queries the first block rows prepare them, one unit's 32
  // columns per workgroup (dispatched first, so their loads overlap the k
  // and v blocks'); the rest are the row slots.
  int by = (int)blockIdx.y;
  if constexpr (SM >= 0) {
    __shared__ __attribute__((aligned(16))) uint16_t qlds[32 * 128];
    if (qp.base) {
      const int q_groups = n_kv * qp.n_rb * (qp.vectors / 32);  // 32-column groups, one workgroup each
      const int qy = (q_groups + (int)gridDim.x - 1) / (int)gridDim.x;
      if (by < qy) {
        const int qw = by * (int)gridDim.x + r;
        prep_q_block<SM>(qw, qw < q_groups, q, n_q, q_w, eps, pos0, sr.rows, qp, wib, lane, qlds);
        return;
      }
      by -= qy;
    }
  }
  const int sy = by * (int)(blockDim.x >> 6) + wib;
  const int n_q_row = (SM >= 0 && qp.base) ? 0 : n_q;
  const int n_slots = SM >= 0 ? n_q_row + n_kv : n_q + 2 * n_kv;
  const int s0 = sy * KS;
  if constexpr (SM >= 0) {
    const int kb = (n_slots + KS - 1) / KS;
    if (sy >= kb + n_kv) return;
    if (sy >= kb) {
      stage_v_quad<T, SM>(v, vp, n_kv, sy - kb, sr, r, lane);
      return;
    }
  } else {
    if (s0 >= n_slots) return;
  }
  if constexpr (SM >= 0) {
    if (r >= sr.rows) {
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const int s = s0 + j;
        if (s < n_q_row || s >= n_slots) continue;
        const int kind = s >= n_q_row + n_kv, h = s - n_q_row - kind * n_kv;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const int i = lane + 64 * p;
          if (i >= half) continue;
          stage_elem<SM>(sr, kind, h, sr.row0 + r, i, 0.f);
          stage_elem<SM>(sr, kind, h, sr.row0 + r, i + half, 0.f);
        }
      }
      return;
    }
  }
  // Source of slot s (q, k or v head of row r); its destination is below.
  auto src = [&](int s) -> const float* {
    if (s < n_q_row) return q + ((size_t)r * n_q + s) * hd;
    if (s < n_q_row + n_kv) return k + ((size_t)r * n_kv + (s - n_q_row)) * hd;
    return v + ((size_t)r * n_kv + (s - n_q_row - n_kv)) * hd;
  };
  // inv_freq first: the sin/cos below wait only for it, not the heads.
  double freq[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) freq[p] = inv.f[min(lane + 64 * p, half - 1)];
  float x0[KS][NP], x1[KS][NP];
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const bool live = s0 + j < n_slots;
    const float* x = src(live ? s0 + j : 0);
    // Unconditional loads from clamped (valid) addresses, so the wait
    // counts stay exact; dead lanes and slots are zeroed afterwards.
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int i = min(lane + 64 * p, half - 1);
      const bool in = live && lane + 64 * p < half;
      const float a0 = x[i], a1 = x[i + half];
      x0[j][p] = in ? a0 : 0.f;
      x1[j][p] = in ? a1 : 0.f;
    }
  }
  float wq0[NP], wq1[NP], wk0[NP], wk1[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int i = min(lane + 64 * p, half - 1);
    wq0[p] = q_w[i];
    wq1[p] = q_w[i + half];
    wk0[p] = k_w[i];
    wk1[p] = k_w[i + half];
  }
  // Every load above is issued before the first use (the scheduler would
  // otherwise sink each head's loads to its arithmetic, one round trip each).
  __builtin_amdgcn_sched_barrier(0);
  const double pos = (double)(pos0 + r);
  // Blocks of v heads only need no angles.
  const bool rotates = s0 < n_q_row + n_kv;
  float sn[NP], cs[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int i = lane + 64 * p;
    double sd = 0.0, cd = 1.0;
    if (qp.rope && i < half) {  // the same f32 values, computed once per position on the host
      cd = qp.rope[(size_t)(pos0 + r) * hd + i];
      sd = qp.rope[(size_t)(pos0 + r) * hd + half + i];
    } else if (rotates && i < half) {
      sincos(pos * freq[p], &sd, &cd);
    }
    sn[p] = (float)sd;
    cs[p] = (float)cd;
    if (tab && sy == 0 && i < half) {
      tab[(size_t)r * hd + i] = cs[p];
      tab[(size_t)r * hd + half + i] = sn[p];
    }
  }
  // The slots' norms first, branch-free within a block that rotates (its v
  // and dead slots compute a norm they do not use), so the f64 reductions
  // and square roots overlap.
  float inv_rms[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    inv_rms[j] = 1.0f;
    if (!rotates) continue;
    double ss = 0.0;
#pragma unroll
    for (int p = 0; p < NP; ++p) ss += (double)x0[j][p] * (double)x0[j][p] + (double)x1[j][p] * (double)x1[j][p];
    ss = wave_sum_f64(ss);
    inv_rms[j] = (float)(1.0 / sqrt(ss / (double)hd + (double)eps));
  }
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const int s = s0 + j;
    if (s >= n_slots) break;
    if (s >= n_q_row + n_kv) {  // v head: copied into the cache
      T* d = vp + ((size_t)r * n_kv + (s - n_q_row - n_kv)) * hd;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int i = lane + 64 * p;
        if (i < half) {
          const float c0 = store_cached<T>(d + i, x0[j][p]);
          const float c1 = store_cached<T>(d + i + half, x1[j][p]);
          if constexpr (SM >= 0) {
            stage_elem<SM>(sr, 1, s - n_q_row - n_kv, sr.row0 + r, i, c0);
            stage_elem<SM>(sr, 1, s - n_q_row - n_kv, sr.row0 + r, i + half, c1);
          }
        }
      }
      continue;
    }
    const bool is_q = s < n_q_row;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int i = lane + 64 * p;
      if (i >= half) continue;
      const float a0 = x0[j][p] * inv_rms[j] * (is_q ? wq0[p] : wk0[p]);
      const float a1 = x1[j][p] * inv_rms[j] * (is_q ? wq1[p] : wk1[p]);
      const float ya = a0 * cs[p] - a1 * sn[p], yb = a0 * sn[p] + a1 * cs[p];
      if (is_q) {
        float* d = q_out + ((size_t)r * n_q + s) * hd;
        d[i] = ya;
        d[i + half] = yb;
      } else {
        T* d = kp + ((size_t)r * n_kv + (s - n_q_row)) * hd;
        const float c0 = store_cached<T>(d + i, ya);
        const float c1 = store_cached<T>(d + i + half, yb);
        if constexpr (SM >= 0) {
          stage_elem<SM>(sr, 0, s - n_q_row, sr.row0 + r, i, c0);
          stage_elem<SM>(sr, 0, s - n_q_row, sr.row0 + r, i + half, c1);
        }
      }
    }
  }
}

template <typename T>
void launch_row_prologue_t(dim3 grid, int np, const float* q, float* q_out, int n_q, const float* k, const float* v,
                           T* kp, T* vp, int n_kv, int hd, const float* q_w, const float* k_w, float eps,
                           const InvFreq& inv, long pos0, float* tab, int sm, const StagedRows& sr, const QPrep& qp,
                           hipStream_t s) {
#define RV_PROLOGUE(NP, SM)                                                                                      \
  hipLaunchKernelGGL((row_prologue_kernel<T, NP, SM>), grid, dim3(SM >= 0 ? 64 * kPrologueWaves : 64), 0, s, q, q_out, \
                     n_q, k, v, kp, vp, n_kv, hd,                                                                \
                     q_w, k_w, eps, inv, pos0, tab, sr, qp)
  if (sm == kF16)
    RV_PROLOGUE(1, kF16);
  else if (sm == kBF16)
    RV_PROLOGUE(1, kBF16);
  else if (np == 1)
    RV_PROLOGUE(1, -1);
  else if (np == 2)
    RV_PROLOGUE(2, -1);
  else
    RV_PROLOGUE(4, -1);
#undef RV_PROLOGUE
}

}  // namespace

HipStatus launch_append(const rv_kv* kv, size_t layer, size_t pos0, const float* k, const float* v, size_t rows,
                        hipStream_t s) {
  HipStatus st;
  if (rows == 0) return st;
  const size_t off = pos0 * kv->kv_dim;
  const dim3 grid((unsigned)rows, (unsigned)kv->n_kv_heads);
  if (kv->elem == RV_ELEM_F32) {
    hipLaunchKernelGGL(append_kernel<float>, grid, dim3(64), 0, s, k, v, (float*)kv->k_layer(layer) + off,
                       (float*)kv->v_layer(layer) + off, (int)kv->kv_dim, (int)kv->head_dim);
  } else {
    hipLaunchKernelGGL(append_kernel<uint16_t>, grid, dim3(64), 0, s, k, v, (uint16_t*)kv->k_layer(layer) + off,
                       (uint16_t*)kv->v_layer(layer) + off, (int)kv->kv_dim, (int)kv->head_dim);
  }
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "append launch";
  return st;
}

HipStatus launch_row_prologue(const rv_kv* kv, size_t layer, size_t cache_row, const float* q, float* q_out,
                              size_t n_q, const float* k, const float* v, size_t rows, const float* q_w,
                              const float* k_w, float eps, const InvFreq& inv, size_t pos0, float* rope_tab,
                              const StageDst* sd, hipStream_t s, const QPrep* qp) {
  HipStatus st;
  if (rows == 0) return st;
  const int hd = (int)kv->head_dim, n_kv = (int)kv->n_kv_heads;
  const int half = hd / 2;
  // Without q heads the kernel still reads its q weights (unused): point
  // them at the k weights.
  if (n_q == 0) q_w = k_w;
  const int np = half <= 64 ? 1 : half <= 128 ? 2 : 4;
  const int n_slots = (int)n_q + 2 * n_kv;
  // Staging: k and v heads only, head_dim 128; the grid covers the chunk's
  // last tile to its end.
  const bool staging = sd && sd->base;
  const bool prep = qp && qp->base;
  // The split mode's tiles are staged whole by the stage kernel (their
  // exponents span all of a tile's rows), never row by row here. q heads
  // run in a staging launch only into the prepared layout.
  if ((prep && (!staging || !qp->rope)) ||
      (staging && ((n_q != 0 && !prep) || hd != 128 || (sd->mode != RV_PREFILL_F16 && sd->mode != RV_PREFILL_BF16)))) {
    st.e = hipErrorInvalidValue;
    st.what = "staged prologue geometry";
    return st;
  }
  const size_t end = cache_row + rows;
  const size_t grid_rows = staging ? rows + (kBT - end % kBT) % kBT : rows;
  const int sm = !staging ? -1 : sd->mode == RV_PREFILL_F16 ? kF16 : kBF16;
  const StagedRows sr{staging ? sd->base : nullptr, staging ? sd->tile_stride : 0, (int)rows, (long)cache_row};
  // Staging: q and k slot blocks, then one block row per v head (its quads
  // of positions along x; grid_rows covers them).
  // Staging: with prepared queries first enough block rows for one
  // workgroup per 32 columns of each unit, then (k blocks + v blocks) /
  // kPrologueWaves.
  int slot_blocks = (n_slots + kSlots - 1) / kSlots;
  if (staging) {
    slot_blocks = (2 * n_kv + kPrologueWaves - 1) / kPrologueWaves;  // a wave per k head, then per v head
    if (prep) {
      const size_t q_groups = (size_t)n_kv * qp->n_rb * (qp->vectors / 32);
      slot_blocks += (int)((q_groups + grid_rows - 1) / grid_rows);
    }
  }
  const QPrep qpv = prep ? *qp : QPrep{};
  const dim3 grid((unsigned)grid_rows, (unsigned)slot_blocks);
  const size_t off = cache_row * kv->kv_dim;
  if (kv->elem == RV_ELEM_F32)
    launch_row_prologue_t<float>(grid, np, q, q_out, (int)n_q, k, v, (float*)kv->k_layer(layer) + off,
                                 (float*)kv->v_layer(layer) + off, n_kv, hd, q_w, k_w, eps, inv, (long)pos0, rope_tab,
                                 sm, sr, qpv, s);
  else
    launch_row_prologue_t<uint16_t>(grid, np, q, q_out, (int)n_q, k, v, (uint16_t*)kv->k_layer(layer) + off,
                                    (uint16_t*)kv->v_layer(layer) + off, n_kv, hd, q_w, k_w, eps, inv, (long)pos0,
                                    rope_tab, sm, sr, qpv, s);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "prologue launch";
  return st;
}

}  // namespace rv
