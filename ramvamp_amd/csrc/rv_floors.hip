// rv_floors.hip — the measurement probes of include/ramvamp_floors.h: an
// empty launch, a plain streaming read, and MFMA issue-rate loops. bench.py
// times them in graphs on the box the attention kernels run on.
#include "../../include/ramvamp_floors.h"
#include "rv_device.hpp"

namespace {

using rv::f16x8;
using rv::f32x16;
using rv::f32x4;

int32_t fail(rv_error* err, int32_t code, uint64_t a, const char* what) {
  if (err) *err = rv_error{code, a, 0, 0, 0, what};
  return code;
}
int32_t done(rv_error* err, const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(err, RV_ERR_HIP, (uint64_t)e, what);
  if (err) *err = rv_error{RV_OK, 0, 0, 0, 0, nullptr};
  return RV_OK;
}

__global__ __launch_bounds__(64) void floor_empty_kernel() {}

// Workgroup b reads 16-byte pieces [lo, hi) of the buffer, eight loads in
// flight per thread (a piece index past hi reads the last piece again, so
// every load is in bounds and the loop has no tail).
__global__ __launch_bounds__(256) void floor_stream_kernel(const f32x4* __restrict__ src, size_t n16,
                                                           float* __restrict__ sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t lo = per * blockIdx.x, hi = lo + per < n16 ? lo + per : n16;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (size_t base = lo + threadIdx.x; base < hi; base += 8 * 256) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const size_t i = base + (size_t)u * 256;
      v[u] = __builtin_nontemporal_load(src + (i < hi ? i : hi - 1));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + (size_t)u * 256 < hi) acc += v[u];
  }
  float s = acc[0] + acc[1] + acc[2] + acc[3];
  s += __shfl_xor(s, 1, 64);
  if (threadIdx.x == 0) sink[blockIdx.x] = s;
}

// FORM 0: 16x16x32 f16, 1: 32x32x16 f16, 2: 16x16x4 f32; C independent
// accumulator chains per wave.
template <int FORM, int C>
__global__ __launch_bounds__(256) void floor_mfma_kernel(uint32_t iters, float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  f16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (_Float16)(0.001f * (float)(lane + e));
    b[e] = (_Float16)(0.002f * (float)(lane - e));
  }
  const float fa = 0.001f * (float)lane, fb = 0.002f * (float)(63 - lane);
  float total = 0.f;
  if constexpr (FORM == 1) {
    f32x16 acc[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
    for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) total += acc[c][r];
  } else {
    f32x4 acc[C];
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if constexpr (FORM == 0)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
        else
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa, fb, acc[c], 0, 0, 0);
      }
#pragma unroll
    for (int c = 0; c < C; ++c) total += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  }
  if (lane == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = total;
}

// MFMA / VALU overlap: 4 independent chains of v_mfma_f32_32x32x16_f16, each
// MFMA followed in issue order by K independent VALU instructions of one
// kind (KIND 0: v_fma_f32, 1: v_exp_f32) on 8 registers; a scheduling fence
// after each chunk keeps that order.
template <int KIND, int K>
__global__ __launch_bounds__(256) void floor_overlap_kernel(uint32_t iters, float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  f16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (_Float16)(0.001f * (float)(lane + e));
    b[e] = (_Float16)(0.002f * (float)(lane - e));
  }
  f32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = 0.25f * (float)(lane + i) / 64.f;
  const float y = 0.999f, z = 0.0001f * (float)lane;
  for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if constexpr (KIND == 0) x[k & 7] = __builtin_fmaf(x[k & 7], y, z);
        else x[k & 7] = __builtin_amdgcn_exp2f(-x[k & 7]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  float total = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) total += acc[c][r];
#pragma unroll
  for (int i = 0; i < 8; ++i) total += x[i];
  if (lane == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = total;
}

template <int KIND>
void launch_overlap(uint32_t k, uint32_t iters, uint32_t n_wg, float* sink, hipStream_t s) {
  switch (k) {
    case 0: hipLaunchKernelGGL((floor_overlap_kernel<KIND, 0>), dim3(n_wg), dim3(256), 0, s, iters, sink); break;
    case 2: hipLaunchKernelGGL((floor_overlap_kernel<KIND, 2>), dim3(n_wg), dim3(256), 0, s, iters, sink); break;
    case 4: hipLaunchKernelGGL((floor_overlap_kernel<KIND, 4>), dim3(n_wg), dim3(256), 0, s, iters, sink); break;
    default: hipLaunchKernelGGL((floor_overlap_kernel<KIND, 8>), dim3(n_wg), dim3(256), 0, s, iters, sink); break;
  }
}

template <int FORM>
void launch_mfma(uint32_t chains, uint32_t iters, uint32_t n_wg, float* sink, hipStream_t s) {
  if (chains == 1)
    hipLaunchKernelGGL((floor_mfma_kernel<FORM, 1>), dim3(n_wg), dim3(256), 0, s, iters, sink);
  else if (chains == 2)
    hipLaunchKernelGGL((floor_mfma_kernel<FORM, 2>), dim3(n_wg), dim3(256), 0, s, iters, sink);
  else
    hipLaunchKernelGGL((floor_mfma_kernel<FORM, 4>), dim3(n_wg), dim3(256), 0, s, iters, sink);
}

}  // namespace

extern "C" {

int32_t rv_floor_empty(void* stream, rv_error* err) {
  hipLaunchKernelGGL(floor_empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream);
  return done(err, "empty launch");
}

int32_t rv_floor_stream_read(const void* src, size_t bytes, uint32_t n_wg, float* sink, void* stream, rv_error* err) {
  if (!src || !sink) return fail(err, RV_ERR_NULL_ARG, 0, !src ? "src" : "sink");
  if (bytes == 0 || bytes % 16 || ((uintptr_t)src & 15))
    return fail(err, RV_ERR_UNSUPPORTED, bytes, "bytes a nonzero multiple of 16, src 16-byte aligned");
  if (n_wg == 0 || n_wg > 65536) return fail(err, RV_ERR_UNSUPPORTED, n_wg, "n_wg in [1, 65536]");
  hipLaunchKernelGGL(floor_stream_kernel, dim3(n_wg), dim3(256), 0, (hipStream_t)stream, (const f32x4*)src,
                     bytes / 16, sink);
  return done(err, "streaming read launch");
}

int32_t rv_floor_mfma(int32_t form, uint32_t chains, uint32_t iters, uint32_t n_wg, float* sink, void* stream,
                      rv_error* err) {
  if (!sink) return fail(err, RV_ERR_NULL_ARG, 0, "sink");
  if (form < 0 || form > 2) return fail(err, RV_ERR_UNSUPPORTED, (uint64_t)form, "form");
  if (chains != 1 && chains != 2 && chains != 4) return fail(err, RV_ERR_UNSUPPORTED, chains, "chains 1, 2 or 4");
  if (iters == 0 || n_wg == 0 || n_wg > 65536) return fail(err, RV_ERR_UNSUPPORTED, n_wg, "iters >= 1, n_wg in [1, 65536]");
  const hipStream_t s = (hipStream_t)stream;
  if (form == RV_FLOOR_MFMA_F16_16X16X32) launch_mfma<0>(chains, iters, n_wg, sink, s);
  else if (form == RV_FLOOR_MFMA_F16_32X32X16) launch_mfma<1>(chains, iters, n_wg, sink, s);
  else launch_mfma<2>(chains, iters, n_wg, sink, s);
  return done(err, "mfma launch");
}

int32_t rv_floor_mfma_valu(int32_t kind, uint32_t valu_per_mfma, uint32_t iters, uint32_t n_wg, float* sink,
                           void* stream, rv_error* err) {
  if (!sink) return fail(err, RV_ERR_NULL_ARG, 0, "sink");
  if (kind != RV_FLOOR_VALU_FMA && kind != RV_FLOOR_VALU_EXP) return fail(err, RV_ERR_UNSUPPORTED, (uint64_t)kind, "kind");
  if (valu_per_mfma != 0 && valu_per_mfma != 2 && valu_per_mfma != 4 && valu_per_mfma != 8)
    return fail(err, RV_ERR_UNSUPPORTED, valu_per_mfma, "valu_per_mfma 0, 2, 4 or 8");
  if (iters == 0 || n_wg == 0 || n_wg > 65536) return fail(err, RV_ERR_UNSUPPORTED, n_wg, "iters >= 1, n_wg in [1, 65536]");
  const hipStream_t s = (hipStream_t)stream;
  if (kind == RV_FLOOR_VALU_FMA) launch_overlap<0>(valu_per_mfma, iters, n_wg, sink, s);
  else launch_overlap<1>(valu_per_mfma, iters, n_wg, sink, s);
  return done(err, "mfma/valu overlap launch");
}

}  // extern "C"
