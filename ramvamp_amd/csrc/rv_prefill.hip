// rv_prefill.hip — causal chunked-prefill attention on gfx950 MFMA.
//
// Replaces scatter_attention -> attention_at_in per row
// (crates/core/src/model/prefill.rs:1322-1408 -> kernels/attention.rs:732):
// query row r of the chunk attends cache positions 0..start+r+1.
//
// Tiling. One workgroup (4 waves) per (kv head, 16-row tile, kv split). The
// tile's query vectors are the 16 rows of every q head of the GQA group, so
// each K/V tile staged in LDS serves all `group` heads: wave w owns heads
// w, w+4, ... (one 16x16 MFMA column block per head). Per 32-position K/V
// tile:
//   S^T[t][m] = sum_d K[t][d] Q[m][d]      (A = K from LDS, B = Q in VGPRs)
//   O^T[d][m] += sum_t V[t][d] P[m][t]     (A = V^T from LDS, B = P in VGPRs)
// on v_mfma_f32_16x16x32_{f16,bf16}. Computing S transposed puts each query
// row's scores in one lane (4 consecutive t per 16x16 block), which is exactly
// the B-operand layout P^T needs, so P never leaves registers.
//
// Arithmetic modes (flags RV_PREFILL_*):
//   EXACT: each operand split as hi + lo f16 (lo = f16(x - hi)); products
//          hi*hi + hi*lo + lo*hi, fp32 accumulate: ~2^-21 relative products,
//          the fp32 parity mode.
//   F16 / BF16: one MFMA per product, fp32 accumulate.
// Softmax is online in fp32 (exp2, log2(e) folded into the score scale).
//
// KV splits (more workgroups than row tiles when the chunk is short) write
// partial (O, max, sum) rows; the last workgroup of a (kv head, row tile) to
// finish merges them with an fp32 log-sum-exp combine.
#include "rv_device.hpp"
#include "rv_internal.hpp"

#include <algorithm>

namespace rv {
namespace {

constexpr int kWG = 256;
constexpr int kD = 128;
constexpr int kBR = 16;          // query rows per tile
constexpr int kBT = 32;          // positions per K/V tile
constexpr int kKPad = kD + 8;    // LDS row stride of K (halves)
constexpr int kVPad = kBT + 8;   // LDS row stride of V^T (halves)
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

// hi = round(x), lo = round(x - hi) (lo only in the split mode).
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

// part layout per (kv head, row tile, split): O[g][m][d] then (max, sum)[g][m]
__host__ __device__ constexpr size_t part_stride(int group) { return (size_t)group * kBR * (kD + 2); }

template <int MODE, typename T, int MT>
__global__ __launch_bounds__(kWG) void prefill_kernel(const float* __restrict__ q, const T* __restrict__ kl,
                                                      const T* __restrict__ vl, int kv_dim, int q_stride,
                                                      int rows, int start, int group, int kv_splits,
                                                      float qscale, float* __restrict__ part,
                                                      unsigned* __restrict__ tickets, float* __restrict__ out) {
  typedef typename Op<MODE>::E E;
  typedef typename Op<MODE>::V8 V8;
  constexpr bool kSplit = Op<MODE>::kSplit;
  constexpr int kPlanes = kSplit ? 2 : 1;

  __shared__ __attribute__((aligned(16))) E k_lds[kPlanes][kBT][kKPad];
  __shared__ __attribute__((aligned(16))) E v_lds[kPlanes][kD][kVPad];

  const int split = blockIdx.x, rt = blockIdx.y, kvh = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lm = lane & 15, kg = lane >> 4;
  const int r0 = rt * kBR;
  const int rows_here = min(kBR, rows - r0);
  const int tile_limit = start + r0 + rows_here;  // positions the last row of the tile sees
  const int n_tt = (tile_limit + kBT - 1) / kBT;
  const int tt_lo = (int)((long)n_tt * split / kv_splits);
  const int tt_hi = (int)((long)n_tt * (split + 1) / kv_splits);

  // This lane's query row (column m of every 16x16 block) and its limit.
  const int my_row = r0 + lm;
  const bool row_ok = my_row < rows;
  const int my_limit = start + my_row + 1;  // attends t < my_limit

  V8 qh[MT][4], ql[MT][4];
  f32x4 o[MT][8];
  float m_run[MT], l_run[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int g = wave + 4 * mt;
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

    // Online softmax per query row (lane column lm); scores for t0 + ts*16 + kg*4 + i.
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

  // Row sums: each lane holds a quarter of its row's positions.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    l_run[mt] += __shfl_xor(l_run[mt], 16, 64);
    l_run[mt] += __shfl_xor(l_run[mt], 32, 64);
  }

  if (kv_splits == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int g = wave + 4 * mt;
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
  float* mine = part + (tile_idx * kv_splits + split) * part_stride(group);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int g = wave + 4 * mt;
    if (g >= group) continue;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[((size_t)g * kBR + lm) * kD + ds * 16 + kg * 4 + i] = o[mt][ds][i];
    if (kg == 0) {
      mine[(size_t)group * kBR * kD + ((size_t)g * kBR + lm) * 2] = m_run[mt];
      mine[(size_t)group * kBR * kD + ((size_t)g * kBR + lm) * 2 + 1] = l_run[mt];
    }
  }
  __threadfence();
  __syncthreads();
  __shared__ unsigned s_last;
  if (tid == 0) s_last = atomicAdd(&tickets[tile_idx], 1u) == (unsigned)(kv_splits - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* base = part + tile_idx * kv_splits * part_stride(group);
  const size_t ml_off = (size_t)group * kBR * kD;
  for (int idx = tid; idx < group * kBR * kD; idx += kWG) {
    const int gm = idx / kD, d = idx % kD;  // gm = g * kBR + m
    const int m = gm % kBR, g = gm / kBR;
    if (r0 + m >= rows) continue;
    float M = kNegSentinel;
    for (int sp = 0; sp < kv_splits; ++sp) M = fmaxf(M, base[sp * part_stride(group) + ml_off + gm * 2]);
    float L = 0.f, O = 0.f;
    for (int sp = 0; sp < kv_splits; ++sp) {
      const float* ps = base + sp * part_stride(group);
      const float a = exp2f(ps[ml_off + gm * 2] - M);
      L += ps[ml_off + gm * 2 + 1] * a;
      O += ps[(size_t)gm * kD + d] * a;
    }
    out[(size_t)(r0 + m) * q_stride + (size_t)(kvh * group + g) * kD + d] = O / L;
  }
  if (tid == 0) __hip_atomic_store(&tickets[tile_idx], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int MODE, typename T>
void launch_mode(int mt, dim3 grid, const float* q, const void* kl, const void* vl, int kv_dim, int q_stride,
                 int rows, int start, int group, int kv_splits, float qscale, float* part, unsigned* tickets,
                 float* out, hipStream_t s) {
  if (mt <= 1)
    hipLaunchKernelGGL((prefill_kernel<MODE, T, 1>), grid, dim3(kWG), 0, s, q, (const T*)kl, (const T*)vl, kv_dim,
                       q_stride, rows, start, group, kv_splits, qscale, part, tickets, out);
  else if (mt == 2)
    hipLaunchKernelGGL((prefill_kernel<MODE, T, 2>), grid, dim3(kWG), 0, s, q, (const T*)kl, (const T*)vl, kv_dim,
                       q_stride, rows, start, group, kv_splits, qscale, part, tickets, out);
  else
    hipLaunchKernelGGL((prefill_kernel<MODE, T, 4>), grid, dim3(kWG), 0, s, q, (const T*)kl, (const T*)vl, kv_dim,
                       q_stride, rows, start, group, kv_splits, qscale, part, tickets, out);
}

template <typename T>
void launch_t(uint32_t mode, int mt, dim3 grid, const float* q, const void* kl, const void* vl, int kv_dim,
              int q_stride, int rows, int start, int group, int kv_splits, float qscale, float* part,
              unsigned* tickets, float* out, hipStream_t s) {
  switch (mode) {
    case RV_PREFILL_F16:
      launch_mode<kF16, T>(mt, grid, q, kl, vl, kv_dim, q_stride, rows, start, group, kv_splits, qscale, part,
                           tickets, out, s);
      break;
    case RV_PREFILL_BF16:
      launch_mode<kBF16, T>(mt, grid, q, kl, vl, kv_dim, q_stride, rows, start, group, kv_splits, qscale, part,
                            tickets, out, s);
      break;
    default:
      launch_mode<kExact, T>(mt, grid, q, kl, vl, kv_dim, q_stride, rows, start, group, kv_splits, qscale, part,
                             tickets, out, s);
  }
}

}  // namespace

bool prefill_supported(size_t head_dim, size_t group) { return head_dim == kD && group >= 1 && group <= 16; }

HipStatus launch_prefill(rv_kv* kv, const float* q_rows, size_t rows, size_t n_q_heads, size_t layer,
                         size_t start, float scale, float* out, uint32_t mode, hipStream_t s) {
  HipStatus st;
  if (rows == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const int n_rt = (int)((rows + kBR - 1) / kBR);
  const int n_kv = (int)kv->n_kv_heads;
  // KV splits: cover the chip (256 CUs) about twice, never below 4 K/V tiles
  // per split for the longest row tile.
  int kv_splits = (int)kv->tune_prefill_kv_split;
  if (kv_splits <= 0) {
    const long longest_tiles = ((long)start + (long)rows + kBT - 1) / kBT;
    kv_splits = (int)std::max<long>(1, std::min<long>((512 + (long)n_rt * n_kv - 1) / ((long)n_rt * n_kv),
                                                      std::max<long>(1, longest_tiles / 4)));
  }
  const size_t n_tiles = (size_t)n_kv * n_rt;
  if (kv_splits > 1) {
    st = ensure_workspace(kv, n_tiles * kv_splits * part_stride(group) * sizeof(float), n_tiles);
    if (st.e != hipSuccess) return st;
  }
  const int mt = (group + 3) / 4;
  const dim3 grid((unsigned)kv_splits, (unsigned)n_rt, (unsigned)n_kv);
  const float qscale = scale * kLog2e;
  const int q_stride = (int)(n_q_heads * kD);
  const uint32_t m = mode & RV_PREFILL_MODE_MASK;
  if (kv->elem == RV_ELEM_F32)
    launch_t<float>(m, mt, grid, q_rows, kv->k_layer(layer), kv->v_layer(layer), (int)kv->kv_dim, q_stride,
                    (int)rows, (int)start, group, kv_splits, qscale, (float*)kv->ws, kv->tickets, out, s);
  else
    launch_t<_Float16>(m, mt, grid, q_rows, kv->k_layer(layer), kv->v_layer(layer), (int)kv->kv_dim, q_stride,
                       (int)rows, (int)start, group, kv_splits, qscale, (float*)kv->ws, kv->tickets, out, s);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "prefill launch";
  return st;
}

}  // namespace rv
