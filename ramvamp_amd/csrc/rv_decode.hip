// rv_decode.hip — single-token GQA decode attention on gfx950.
//
// Replaces attention_body / qk_scores / softmax / v_reduce
// (crates/core/src/kernels/attention.rs:1075-1303) for the decode and
// position-limited forms.
//
// Fast path (head_dim 128, group 1/2/4/8): one workgroup per (kv head,
// split of the position axis). A K or V row's 128-element head slice is read
// by one 16-lane group, 8 elements (16 or 32 bytes) per lane, and serves the
// whole GQA group from registers: every K and V byte is loaded once per call.
// QK dots reduce over the 16 lanes with DPP; softmax is online (running max
// and sum per query head, exp2 with log2(e) folded into q); the splits of one
// kv head are merged by the last workgroup to finish (an atomic ticket) with
// an fp32 log-sum-exp combine.
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

constexpr int kWG = 256;                    // 4 waves
constexpr int kD = 128;                     // head_dim of the fast path
constexpr int kLPR = 16;                    // lanes per K/V row (8 elements each)
constexpr int kRowsPerStep = kWG / kLPR;    // 16 rows per workgroup step
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegSentinel = -1.0e30f;    // finite "no position yet" max

template <int G>
struct PartLayout {
  // per (kv head, split): o[G][kD] then (m, l) per head
  static constexpr int kStride = G * (kD + 2);
};

template <typename T, int G, int R>
__global__ __launch_bounds__(kWG) void decode_split_kernel(const float* __restrict__ q,
                                                           const T* __restrict__ kl,
                                                           const T* __restrict__ vl, int kv_dim,
                                                           int positions, int split_len,
                                                           int n_splits, int kv_lo, float qscale,
                                                           float* __restrict__ part,
                                                           unsigned* __restrict__ tickets,
                                                           float* __restrict__ out) {
  const int split = blockIdx.x;
  const int hidx = blockIdx.y;  // kv head within the range
  const int kvh = kv_lo + hidx;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & (kLPR - 1);
  const int row = wave * (64 / kLPR) + (lane >> 4);  // 0..15
  const int t_begin = split * split_len;
  const int t_end = min(positions, t_begin + split_len);

  float qr[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qp = q + (size_t)(kvh * G + g) * kD + c * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) qr[g][e] = qp[e] * qscale;
  }
  float o[G][8], m[G], l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegSentinel;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }

  const size_t col = (size_t)kvh * kD + c * 8;
  for (int t0 = t_begin; t0 < t_end; t0 += R * kRowsPerStep) {
    float kx[R][8], vx[R][8];
    bool valid[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int t = t0 + j * kRowsPerStep + row;
      valid[j] = t < t_end;
      if (valid[j]) {
        load8(kl + (size_t)t * kv_dim + col, kx[j]);
        load8(vl + (size_t)t * kv_dim + col, vx[j]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) kx[j][e] = vx[j][e] = 0.f;
      }
    }
    float s[R][G];
#pragma unroll
    for (int j = 0; j < R; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += qr[g][e] * kx[j][e];
        acc = group_sum<kLPR>(acc);
        s[j][g] = valid[j] ? acc : -INFINITY;
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
  }

  // Merge the four row groups of this wave (lanes 16 and 32 apart).
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off, 64);
      const float lo = __shfl_xor(l[g], off, 64);
      const float mn = fmaxf(m[g], mo);
      const float a = exp2f(m[g] - mn), b = exp2f(mo - mn);
      l[g] = l[g] * a + lo * b;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] = o[g][e] * a + __shfl_xor(o[g][e], off, 64) * b;
      m[g] = mn;
    }
  }

  __shared__ float sm_o[4][G][kD];
  __shared__ float sm_ml[4][G][2];
  if (lane < kLPR) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_o[wave][g][c * 8 + e] = o[g][e];
      if (c == 0) {
        sm_ml[wave][g][0] = m[g];
        sm_ml[wave][g][1] = l[g];
      }
    }
  }
  __syncthreads();

  float* mine = part + ((size_t)hidx * n_splits + split) * PartLayout<G>::kStride;
  for (int idx = tid; idx < G * kD; idx += kWG) {
    const int g = idx / kD, d = idx % kD;
    float M = sm_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, sm_ml[w][g][0]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = exp2f(sm_ml[w][g][0] - M);
      L += sm_ml[w][g][1] * a;
      O += sm_o[w][g][d] * a;
    }
    if (n_splits == 1) {
      out[(size_t)(hidx * G + g) * kD + d] = O / L;
    } else {
      mine[g * kD + d] = O;
      if (d == 0) {
        mine[G * kD + 2 * g] = M;
        mine[G * kD + 2 * g + 1] = L;
      }
    }
  }
  if (n_splits == 1) return;

  // Last workgroup of this kv head merges every split.
  __threadfence();
  __syncthreads();
  __shared__ unsigned s_last;
  if (tid == 0) {
    const unsigned prev = atomicAdd(&tickets[hidx], 1u);
    s_last = prev == (unsigned)(n_splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const float* base = part + (size_t)hidx * n_splits * PartLayout<G>::kStride;
  for (int idx = tid; idx < G * kD; idx += kWG) {
    const int g = idx / kD, d = idx % kD;
    float M = kNegSentinel;
    for (int s = 0; s < n_splits; ++s) M = fmaxf(M, base[(size_t)s * PartLayout<G>::kStride + G * kD + 2 * g]);
    float L = 0.f, O = 0.f;
#pragma unroll 4
    for (int s = 0; s < n_splits; ++s) {
      const float* ps = base + (size_t)s * PartLayout<G>::kStride;
      const float a = exp2f(ps[G * kD + 2 * g] - M);
      L += ps[G * kD + 2 * g + 1] * a;
      O += ps[g * kD + d] * a;
    }
    out[(size_t)(hidx * G + g) * kD + d] = O / L;
  }
  if (tid == 0) __hip_atomic_store(&tickets[hidx], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

template <typename T, int G, int R>
void launch_split(const rv_kv* kv, const float* q, const void* kl, const void* vl, int positions,
                  int split_len, int n_splits, int kv_lo, int n_heads, float qscale, float* part,
                  unsigned* tickets, float* out, hipStream_t s) {
  hipLaunchKernelGGL((decode_split_kernel<T, G, R>), dim3(n_splits, n_heads), dim3(kWG), 0, s, q,
                     (const T*)kl, (const T*)vl, (int)kv->kv_dim, positions, split_len, n_splits,
                     kv_lo, qscale, part, tickets, out);
}

template <typename T, int G>
void launch_split_r(const rv_kv* kv, const float* q, const void* kl, const void* vl, int positions,
                    int split_len, int n_splits, int kv_lo, int n_heads, float qscale, float* part,
                    unsigned* tickets, float* out, hipStream_t s) {
  const int steps = split_len / kRowsPerStep;
  if (steps >= 4)
    launch_split<T, G, 4>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s);
  else if (steps >= 2)
    launch_split<T, G, 2>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s);
  else
    launch_split<T, G, 1>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s);
}

template <typename T>
bool launch_split_g(int group, const rv_kv* kv, const float* q, const void* kl, const void* vl,
                    int positions, int split_len, int n_splits, int kv_lo, int n_heads, float qscale,
                    float* part, unsigned* tickets, float* out, hipStream_t s) {
  switch (group) {
    case 1: launch_split_r<T, 1>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s); return true;
    case 2: launch_split_r<T, 2>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s); return true;
    case 4: launch_split_r<T, 4>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s); return true;
    case 8: launch_split_r<T, 8>(kv, q, kl, vl, positions, split_len, n_splits, kv_lo, n_heads, qscale, part, tickets, out, s); return true;
    default: return false;
  }
}

}  // namespace

// Positions per split: enough workgroups to cover the chip about twice
// (256 CUs) with at least 32 and at most 1024 positions each, rounded to the
// 16-row workgroup step.
static int pick_split_len(const rv_kv* kv, int positions, int n_heads) {
  if (kv->tune_decode_split_len > 0) return (int)((kv->tune_decode_split_len + 15) / 16 * 16);
  const long target_wgs = 512;
  long per = ((long)positions * n_heads + target_wgs - 1) / target_wgs;
  per = std::max<long>(32, std::min<long>(1024, per));
  return (int)((per + 15) / 16 * 16);
}

HipStatus launch_decode(rv_kv* kv, const float* q, size_t n_q_heads, size_t layer, size_t positions,
                        float scale, size_t kv_lo, size_t kv_hi, float* out, hipStream_t s) {
  HipStatus st;
  const int n_heads = (int)(kv_hi - kv_lo);
  if (n_heads == 0) return st;
  const int group = (int)(n_q_heads / kv->n_kv_heads);
  const void* kl = kv->k_layer(layer);
  const void* vl = kv->v_layer(layer);
  const bool fast = kv->head_dim == kD && (group == 1 || group == 2 || group == 4 || group == 8);
  if (fast) {
    const int split_len = pick_split_len(kv, (int)positions, n_heads);
    const int n_splits = (int)((positions + split_len - 1) / split_len);
    const size_t part_bytes = (size_t)n_heads * n_splits * group * (kD + 2) * sizeof(float);
    st = ensure_workspace(kv, part_bytes, (size_t)n_heads);
    if (st.e != hipSuccess) return st;
    const float qscale = scale * kLog2e;
    bool ok;
    if (kv->elem == RV_ELEM_F32)
      ok = launch_split_g<float>(group, kv, q, kl, vl, (int)positions, split_len, n_splits, (int)kv_lo, n_heads,
                                 qscale, (float*)kv->ws, kv->tickets, out, s);
    else
      ok = launch_split_g<_Float16>(group, kv, q, kl, vl, (int)positions, split_len, n_splits, (int)kv_lo,
                                    n_heads, qscale, (float*)kv->ws, kv->tickets, out, s);
    (void)ok;
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
