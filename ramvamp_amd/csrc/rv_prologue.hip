// rv_prologue.hip — per-head QK-RMSNorm + NeoX RoPE and the KV append.
//
// Replaces, per token row, rmsnorm_in_place over each head
// (crates/core/src/kernels/primitives/norm.rs:18-26, :72-90), rope_neox_heads
// (primitives/rope.rs:31-45, :82-105) and KvCache::append (kv/mod.rs:336-368),
// as called at model/forward.rs:2622-2631 and model/prefill.rs:2057-2087.
//
// One wavefront per (row, head). The f32 arithmetic is the reference's, op
// for op and with contraction off: `x * inv * w` left to right, the rotation
// as two separately rounded products and a subtraction/addition. The mean of
// squares is summed in f64 (a tree, not the reference's sequential order: the
// two agree to f64 rounding before the cast to f32). RoPE angles are
// `pos * inv_freq` in f64 with inv_freq computed on the host in f64, then
// sin/cos in f64 and cast to f32, as rope.rs:35-39 does.
#include "rv_device.hpp"
#include "rv_internal.hpp"

#include <math.h>

namespace rv {

void fill_inv_freq(InvFreq& t, size_t head_dim, float theta) {
  const double base = (double)theta;
  const double dim = (double)head_dim;
  for (size_t i = 0; i < head_dim / 2 && i < (size_t)kMaxHalf; ++i) t.f[i] = pow(base, -2.0 * (double)i / dim);
}

namespace {

// Normalise (optional) and rotate one head of `hd` elements held in `x`
// (global memory, read once), returning the results through `emit(i, y)`.
template <typename Emit>
__device__ __forceinline__ void norm_rope_head(const float* __restrict__ x, int hd, const float* __restrict__ w,
                                               float eps, bool norm, const InvFreq& inv, double pos, Emit emit) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int half = hd / 2;
  float inv_rms = 1.0f;
  if (norm) {
    double ss = 0.0;
    for (int i = lane; i < hd; i += 64) {
      const double v = (double)x[i];
      ss += v * v;
    }
    ss = wave_sum_f64(ss);
    const double mean = ss / (double)hd;
    inv_rms = (float)(1.0 / sqrt(mean + (double)eps));
  }
  for (int i = lane; i < half; i += 64) {
    float x0 = x[i], x1 = x[i + half];
    if (norm) {
      x0 = x0 * inv_rms * w[i];
      x1 = x1 * inv_rms * w[i + half];
    }
    const double ang = pos * inv.f[i];
    const float sn = (float)sin(ang), cs = (float)cos(ang);
    const float a = x0 * cs, b = x1 * sn, c = x0 * sn, d = x1 * cs;
    emit(i, a - b);
    emit(i + half, c + d);
  }
}

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

// grid (rows, n_kv_heads), one wave each: K head normalised + rotated (or
// copied), V head copied, both converted to the plane's element type.
template <typename T>
__global__ __launch_bounds__(64) void append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                    T* __restrict__ kp, T* __restrict__ vp, int kv_dim, int hd,
                                                    bool norm, const float* __restrict__ k_w, float eps,
                                                    InvFreq inv, long pos0) {
  const int r = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x;
  const size_t src = (size_t)r * kv_dim + (size_t)h * hd;
  T* kd = kp + src;
  T* vd = vp + src;
  if (norm) {
    norm_rope_head(k + src, hd, k_w, eps, true, inv, (double)(pos0 + r),
                   [&](int i, float y) { store_elem<T>(kd + i, y); });
  } else {
    for (int i = lane; i < hd; i += 64) store_elem<T>(kd + i, k[src + i]);
  }
  for (int i = lane; i < hd; i += 64) store_elem<T>(vd + i, v[src + i]);
}

__global__ __launch_bounds__(64) void q_prologue_kernel(const float* __restrict__ q, float* __restrict__ q_out,
                                                        int n_heads, int hd, const float* __restrict__ w, float eps,
                                                        InvFreq inv, long pos0) {
  const int r = blockIdx.x, h = blockIdx.y;
  const size_t off = ((size_t)r * n_heads + h) * hd;
  float* dst = q_out + off;
  norm_rope_head(q + off, hd, w, eps, true, inv, (double)(pos0 + r), [&](int i, float y) { dst[i] = y; });
}

}  // namespace

HipStatus launch_append(const rv_kv* kv, size_t layer, size_t pos0, const float* k, const float* v, size_t rows,
                        bool norm, const float* k_w, float eps, const InvFreq* inv, hipStream_t s) {
  HipStatus st;
  if (rows == 0) return st;
  const size_t off = pos0 * kv->kv_dim;
  static const InvFreq kZero = {};
  const InvFreq& f = inv ? *inv : kZero;
  const dim3 grid((unsigned)rows, (unsigned)kv->n_kv_heads);
  if (kv->elem == RV_ELEM_F32) {
    hipLaunchKernelGGL(append_kernel<float>, grid, dim3(64), 0, s, k, v, (float*)kv->k_layer(layer) + off,
                       (float*)kv->v_layer(layer) + off, (int)kv->kv_dim, (int)kv->head_dim, norm, k_w, eps, f,
                       (long)pos0);
  } else {
    hipLaunchKernelGGL(append_kernel<uint16_t>, grid, dim3(64), 0, s, k, v, (uint16_t*)kv->k_layer(layer) + off,
                       (uint16_t*)kv->v_layer(layer) + off, (int)kv->kv_dim, (int)kv->head_dim, norm, k_w, eps,
                       f, (long)pos0);
  }
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "append launch";
  return st;
}

HipStatus launch_q_prologue(const float* q, float* q_out, size_t rows, size_t n_heads, size_t head_dim,
                            const float* w, float eps, const InvFreq& inv, size_t pos0, hipStream_t s) {
  HipStatus st;
  if (rows == 0) return st;
  hipLaunchKernelGGL(q_prologue_kernel, dim3((unsigned)rows, (unsigned)n_heads), dim3(64), 0, s, q, q_out,
                     (int)n_heads, (int)head_dim, w, eps, inv, (long)pos0);
  st.e = hipGetLastError();
  if (st.e != hipSuccess) st.what = "q prologue launch";
  return st;
}

}  // namespace rv
