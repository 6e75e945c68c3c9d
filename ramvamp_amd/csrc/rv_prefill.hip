// rv_prefill.hip — causal chunked-prefill attention on gfx950 MFMA.
//
// Replaces scatter_attention -> attention_at_in per row
// (crates/core/src/model/prefill.rs:1322-1408 -> kernels/attention.rs:732):
// query row r of the chunk attends cache positions 0..start+r+1.
//
// Tiling. One workgroup (4 waves) per (kv head, tile of ROWS query rows, kv
// split). The tile's query vectors are its ROWS rows of every q head of the
// GQA group, so each K/V tile staged in LDS serves all `group` heads. A 16x16
// MFMA column block holds 16/ROWS heads x ROWS rows; wave w owns column
// blocks w, w+4, .... Per 32-position K/V tile:
//   S^T[t][m] = sum_d K[t][d] Q[m][d]      (A = K from LDS, B = Q in VGPRs)
//   O^T[d][m] += sum_t V[t][d] P[m][t]     (A = V^T from LDS, B = P in VGPRs)
// on v_mfma_f32_16x16x32_{f16,bf16}. Computing S transposed puts each query
// vector's scores in one lane (4 consecutive t per 16x16 block), which is
// exactly the B-operand layout P^T needs, so P never leaves registers.
//
// Arithmetic modes (flags RV_PREFILL_*):
//   EXACT: each operand split as hi + lo f16 (lo = f16(x - hi)); products
//          hi*hi + hi*lo + lo*hi, fp32 accumulate: ~2^-21 relative products,
//          the fp32 parity mode.
//   F16 / BF16: one MFMA per product, fp32 accumulate.
// Softmax is online in fp32 (exp2, log2(e) folded into the score scale).
//
// KV splits are used only when the row tiles alone leave most of the chip
// idle (short chunks): each split writes partial (O, max, sum) rows and the
// last workgroup of a (kv head, row tile) to finish merges them, with split
// maxima and weights staged in LDS and 16-byte partial loads.
#include "rv_device.hpp"
#include "rv_internal.hpp"

#include <algorithm>

namespace rv {
namespace {

constexpr int kWG = 256;
constexpr int kD = 128;
constexpr int kBT = 32;          // positions per K/V tile
constexpr int kKPad = kD + 8;    // LDS row stride of K (halves)
constexpr int kVPad = kBT + 8;   // LDS row stride of V^T (halves)
constexpr int kMaxKvSplits = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegSentinel = -1.0e30f;

enum Mode { kExact = 0, kF16 = 1, kBF16 = 2 };

template <int MODE>
struct Op;
template <>
struct Op<kExact> {
  typedef _Float16 E;
  typedef f16x8 V8;
  static constexpr bool kSplit = true;
  __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <>
struct Op<kF16> {
  typedef _Float16 E;
  typedef f16x8 V8;
  static constexpr bool kSplit = false;
  __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <>
struct Op<kBF16> {
  typedef __bf16 E;
  typedef bf16x8 V8;
  static constexpr bool kSplit = false;
  __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

// hi = round(x), lo = round(x - hi) (lo only matters in the split mode).
template <typename E>
__device__ __forceinline__ void split2(float x, E& hi, E& lo) {
  hi = (E)x;
  lo = (E)(x - (float)hi);
}

template <typename T>
__device__ __forceinline__ void load16(const T* p, float (&x)[16]);
template <>
__device__ __forceinline__ void load16<float>(const float* p, float (&x)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x4 a = reinterpret_cast<const f32x4*>(p)[i];
    x[4 * i] = a[0];
    x[4 * i + 1] = a[1];
    x[4 * i + 2] = a[2];
    x[4 * i + 3] = a[3];
  }
}
template <>
__device__ __forceinline__ void load16<_Float16>(const _Float16* p, float (&x)[16]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    f16x8 a = reinterpret_cast<const f16x8*>(p)[i];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[8 * i + j] = (float)a[j];
  }
}

// Partial layout per (kv head, row tile, split): O[g][r][d], then (max, sum)[g][r],
// padded to a 16-byte multiple.
__host__ __device__ constexpr size_t part_stride(int group, int rows) {
  return (size_t)group * rows * kD + ((size_t)2 * group * rows + 3) / 4 * 4;
}

template <int MODE, typename T, int MT, int ROWS>
__global__ __launch_bounds__(kWG) void prefill_kernel(const float* __restrict__ q, const T* __restrict__ kl,
                                                      const T* __restrict__ vl, int kv_dim, int q_stride,
                                                      int rows, int start, int group, int kv_splits,
                                                      float qscale, float* __restrict__ part,
                                                      unsigned* __restrict__ tickets, float* __restrict__ out) {
  typedef typename Op<MODE>::E E;
  typedef typename Op<MODE>::V8 V8;
  constexpr bool kSplit = Op<MODE>::kSplit;
  constexpr int kPlanes = kSplit ? 2 : 1;
  constexpr int HPT = 16 / ROWS;  // heads per 16-column block

  __shared__ __attribute__((aligned(16))) E k_lds[kPlanes][kBT][kKPad];
  __shared__ __attribute__((aligned(16))) E v_lds[kPlanes][kD][kVPad];

  const int split = blockIdx.x, rt = blockIdx.y, kvh = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lm = lane & 15, kg = lane >> 4;
  const int r0 = rt * ROWS;
  const int rows_here = min(ROWS, rows - r0);
  const int tile_limit = start + r0 + rows_here;  // positions the last row of the tile sees
  const int n_tt = (tile_limit + kBT - 1) / kBT;
  const int tt_lo = (int)((long)n_tt * split / kv_splits);
  const int tt_hi = (int)((long)n_tt * (split + 1) / kv_splits);

  // This lane's query vector (column lm of every 16x16 block): a row and a
  // head offset inside the block.
  const int rsub = lm % ROWS, hsub = lm / ROWS;
  const int my_row = r0 + rsub;
  const bool row_ok = my_row < rows;
  const int my_limit = start + my_row + 1;  // attends t < my_limit

  V8 qh[MT][4], ql[MT][4];
  f32x4 o[MT][8];
  float m_run[MT], l_run[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int g = (wave + 4 * mt) * HPT + hsub;
    const bool g_ok = g < group && row_ok;
    const float* qp = q + (size_t)my_row * q_stride + (size_t)(kvh * group + g) * kD;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = g_ok ? qp[ds * 32 + kg * 8 + j] : 0.f;
        E hi, lo;
        split2(x, hi, lo);
        qh[mt][ds][j] = hi;
        ql[mt][ds][j] = lo;
      }
    }
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) o[mt][ds] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[mt] = kNegSentinel;
    l_run[mt] = 0.f;
  }

  // K/V tile loader mapping: thread -> (position, 16-element d chunk).
  const int ld_t = tid >> 3, ld_d = (tid & 7) * 16;

  for (int tt = tt_lo; tt < tt_hi; ++tt) {
    const int t0 = tt * kBT;
    __syncthreads();
    {
      const int t = t0 + ld_t;
      float kx[16], vx[16];
      if (t < tile_limit) {
        load16<T>(kl + (size_t)t * kv_dim + (size_t)kvh * kD + ld_d, kx);
        load16<T>(vl + (size_t)t * kv_dim + (size_t)kvh * kD + ld_d, vx);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) kx[i] = vx[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        E kh, klo, vh, vlo;
        split2(kx[i], kh, klo);
        split2(vx[i], vh, vlo);
        k_lds[0][ld_t][ld_d + i] = kh;
        v_lds[0][ld_d + i][ld_t] = vh;
        if constexpr (kSplit) {
          k_lds[kPlanes - 1][ld_t][ld_d + i] = klo;
          v_lds[kPlanes - 1][ld_d + i][ld_t] = vlo;
        }
      }
    }
    __syncthreads();

    // S^T for both 16-position halves of the tile.
    f32x4 s[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) s[mt][0] = s[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) {
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const V8 a = *reinterpret_cast<const V8*>(&k_lds[0][ts * 16 + lm][ds * 32 + kg * 8]);
        V8 alo;
        if constexpr (kSplit) alo = *reinterpret_cast<const V8*>(&k_lds[kPlanes - 1][ts * 16 + lm][ds * 32 + kg * 8]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          s[mt][ts] = Op<MODE>::mfma(a, qh[mt][ds], s[mt][ts]);
          if constexpr (kSplit) {
            s[mt][ts] = Op<MODE>::mfma(alo, qh[mt][ds], s[mt][ts]);
            s[mt][ts] = Op<MODE>::mfma(a, ql[mt][ds], s[mt][ts]);
          }
        }
      }
    }

    // Online softmax per query vector (lane column lm); scores for t0 + ts*16 + kg*4 + i.
    V8 pb[MT], pl[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float sv[8];
      float mx = kNegSentinel;
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t0 + ts * 16 + kg * 4 + i;
          const float x = (t < my_limit) ? s[mt][ts][i] * qscale : -INFINITY;
          sv[ts * 4 + i] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m_run[mt], mx);
      const float alpha = exp2f(m_run[mt] - mn);
      m_run[mt] = mn;
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = exp2f(sv[j] - mn);
        psum += p;
        E hi, lo;
        split2(p, hi, lo);
        pb[mt][j] = hi;
        pl[mt][j] = lo;
      }
      l_run[mt] = l_run[mt] * alpha + psum;
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) o[mt][ds] *= alpha;
    }

    // O^T += V^T P^T: A row d = ds*16 + lm, slots t = kg*4 + {0..3} and 16 + kg*4 + {0..3}.
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
      V8 a, alo;
      {
        const E* vr = &v_lds[0][ds * 16 + lm][0];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = vr[kg * 4 + i];
          a[4 + i] = vr[16 + kg * 4 + i];
        }
        if constexpr (kSplit) {
          const E* vl2 = &v_lds[kPlanes - 1][ds * 16 + lm][0];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            alo[i] = vl2[kg * 4 + i];
            alo[4 + i] = vl2[16 + kg * 4 + i];
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        o[mt][ds] = Op<MODE>::mfma(a, pb[mt], o[mt][ds]);
        if constexpr (kSplit) {
          o[mt][ds] = Op<MODE>::mfma(alo, pb[mt], o[mt][ds]);
          o[mt][ds] = Op<MODE>::mfma(a, pl[mt], o[mt][ds]);
        }
      }
    }
  }

  // Row sums: each lane holds a quarter of its vector's positions.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    l_run[mt] += __shfl_xor(l_run[mt], 16, 64);
    l_run[mt] += __shfl_xor(l_run[mt], 32, 64);
  }

  if (kv_splits == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int g = (wave + 4 * mt) * HPT + hsub;
      if (g >= group || !row_ok) continue;
      const float inv = 1.0f / l_run[mt];
      float* op = out + (size_t)my_row * q_stride + (size_t)(kvh * group + g) * kD;
#pragma unroll
      for (int ds = 0; ds < 8; ++ds)
#pragma unroll
        for (int i = 0; i < 4; ++i) op[ds * 16 + kg * 4 + i] = o[mt][ds][i] * inv;
    }
    return;
  }

  // Partial (O, max, sum) for this split.
  const int n_rt = gridDim.y;
  const size_t tile_idx = (size_t)kvh * n_rt + rt;
  const size_t stride = part_stride(group, ROWS);
  const size_t ml_off = (size_t)group * ROWS * kD;
  float* mine = part + (tile_idx * kv_splits + split) * stride;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int g = (wave + 4 * mt) * HPT + hsub;
    if (g >= group) continue;
    const size_t v = (size_t)g * ROWS + rsub;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
      *reinterpret_cast<f32x4*>(&mine[v * kD + ds * 16 + kg * 4]) = o[mt][ds];
    if (kg == 0) {
      mine[ml_off + v * 2] = m_run[mt];
      mine[ml_off + v * 2 + 1] = l_run[mt];
    }
  }
  __threadfence();
  __syncthreads();
  __shared__ unsigned s_last;
  if (tid == 0) s_last = atomicAdd(&tickets[tile_idx], 1u) == (unsigned)(kv_splits - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // Merge: split weights per query vector in LDS, then 16-byte partial rows.
  const float* base = part + tile_idx * kv_splits * stride;
  const int nv = group * ROWS;  // query vectors of the tile
  __shared__ float sm_w[kMaxKvSplits][16 * 16];
  __shared__ float sm_inv[16 * 16];
  for (int v = tid; v < nv; v += kWG) {
    float M = kNegSentinel;
    for (int sp = 0; sp < kv_splits; ++sp) M = fmaxf(M, base[sp * stride + ml_off + v * 2]);
    float L = 0.f;
    for (int sp = 0; sp < kv_splits; ++sp) {
      const float w = exp2f(base[sp * stride + ml_off + v * 2] - M);
      sm_w[sp][v] = w;
      L += w * base[sp * stride + ml_off + v * 2 + 1];
    }
    sm_inv[v] = 1.0f / L;
  }
  __syncthreads();
  for (int idx = tid; idx < nv * (kD / 4); idx += kWG) {
    const int v = idx / (kD / 4), d = (idx % (kD / 4)) * 4;
    const int g = v / ROWS, r = v % ROWS;
    if (r0 + r >= rows) continue;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < kv_splits; ++sp)
      O += *reinterpret_cast<const f32x4*>(&base[sp * stride + (size_t)v * kD + d]) * sm_w[sp][v];
    O *= sm_inv[v];
    float* op = out + (size_t)(r0 + r) * q_stride + (size_t)(kvh * group + g) * kD + d;
#pragma unroll
    for (int i = 0; i < 4; ++i) op[i] = O[i];
  }
  if (tid == 0) __hip_atomic_store(&tickets[tile_idx], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct PrefillArgs {
  dim3 grid;
  const float* q;
  const void* kl;
  const void* vl;
  int kv_dim, q_stride, rows, start, group, kv_splits;
  float qscale;
  float* part;
  unsigned* tickets;
  float* out;
  TimedPair tp;
};

template <int MODE, typename T, int MT, int ROWS>
void launch_one(const PrefillArgs& a, hipStream_t s) {
  launch_timed(a.tp, prefill_kernel<MODE, T, MT, ROWS>, a.grid, dim3(kWG), s, a.q, (const T*)a.kl, (const T*)a.vl,
               a.kv_dim, a.q_stride, a.rows, a.start, a.group, a.kv_splits, a.qscale, a.part, a.tickets, a.out);
}

// MT = column blocks per wave = ceil(group * ROWS / 16 / 4).
template <int MODE, typename T, int ROWS>
void launch_rows(int mt, const PrefillArgs& a, hipStream_t s) {
  if (mt <= 1)
    launch_one<MODE, T, 1, ROWS>(a, s);
  else if (mt == 2)
    launch_one<MODE, T, 2, ROWS>(a, s);
  else
    launch_one<MODE, T, 4, ROWS>(a, s);
}

template <int MODE, typename T>
void launch_mode(int rows_per_tile, int mt, const PrefillArgs& a, hipStream_t s) {
  if (rows_per_tile == 8)
    launch_rows<MODE, T, 8>(mt, a, s);
  else
    launch_rows<MODE, T, 16>(mt, a, s);
}

template <typename T>
void launch_t(uint32_t mode, int rows_per_tile, int mt, const PrefillArgs& a, hipStream_t s) {
  switch (mode) {
    case RV_PREFILL_F16: launch_mode<kF16, T>(rows_per_tile, mt, a, s); break;
    case RV_PREFILL_BF16: launch_mode<kBF16, T>(rows_per_tile, mt, a, s); break;
    default: launch_mode<kExact, T>(rows_per_tile, mt, a, s);
  }
}

}  // namespace

bool prefill_supported(size_t head_dim, size_t group) { return head_dim == kD && group >= 1 && group <= 16; }

HipStatus launch_prefill(rv_kv* kv, const float* q_rows, size_t rows, size_t n_q_heads, size_t layer,
                         size_t start, float scale, float* out, uint32_t mode, hipStream_t s) {
  HipStatus st;
  if (rows == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const int n_kv = (int)kv->n_kv_heads;
  // Row tiles of 8 (two heads per MFMA column block) when the group is even,
  // so a 512-row chunk fills the chip without splitting the KV axis.
  int rows_per_tile = (kv->tune_prefill_rows == 16 || group % 2) ? 16 : 8;
  if (kv->tune_prefill_rows == 8 && group % 2 == 0) rows_per_tile = 8;
  const int n_rt = (int)((rows + rows_per_tile - 1) / rows_per_tile);
  const int mt = (group * rows_per_tile / 16 + 3) / 4;
  int kv_splits = (int)kv->tune_prefill_kv_split;
  if (kv_splits <= 0) {
    // Split the KV axis only when the tiles cover under half the chip, and
    // keep at least 4 K/V tiles per split.
    const long tiles = (long)n_rt * n_kv;
    const long longest = ((long)start + (long)rows + kBT - 1) / kBT;
    kv_splits = tiles >= 128 ? 1 : (int)std::min<long>(256 / tiles, std::max<long>(1, longest / 4));
  }
  kv_splits = std::max(1, std::min(kv_splits, kMaxKvSplits));
  const size_t n_tiles = (size_t)n_kv * n_rt;
  if (kv_splits > 1) {
    st = ensure_workspace(kv, n_tiles * kv_splits * part_stride(group, rows_per_tile) * sizeof(float), n_tiles);
    if (st.e != hipSuccess) return st;
  }
  PrefillArgs a{dim3((unsigned)kv_splits, (unsigned)n_rt, (unsigned)n_kv), q_rows, kv->k_layer(layer),
                kv->v_layer(layer), (int)kv->kv_dim, (int)(n_q_heads * kD), (int)rows, (int)start, group,
                kv_splits, scale * kLog2e, (float*)kv->ws, kv->tickets, out, timing_pair(kv, s)};
  const uint32_t m = mode & RV_PREFILL_MODE_MASK;
  if (kv->elem == RV_ELEM_F32)
    launch_t<float>(m, rows_per_tile, mt, a, s);
  else
    launch_t<_Float16>(m, rows_per_tile, mt, a, s);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "prefill launch";
  return st;
}

}  // namespace rv
