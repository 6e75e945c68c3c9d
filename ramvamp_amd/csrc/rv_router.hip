// rv_router.hip — the MoE router's decision (include/ramvamp_router.h;
// model/forward.rs:2658-2705), bit for bit.
//
// One workgroup per row. The row is staged in LDS; thread e computes expert
// e's logit as dot_f32 does (forward.rs:1231-1238): one serial f32 sum,
// each product rounded before it is added (contraction off), in index
// order. The softmax (softmax.rs:18-40) takes the max over the logits, each
// thread its exponential in f64, and one thread the f64 sum in expert order
// (the reference's order) and the f32 reciprocal; the same thread then runs
// the reference's top-k scan (strict >, so the first index wins ties; the
// winner set to -inf) and the renormalization (an f32 sum in selection
// order, then one division each).
#include <hip/hip_runtime.h>

#include "../../include/ramvamp_router.h"
#include "rv_internal.hpp"

namespace rv {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxExperts = 1024;
constexpr int kMaxHidden = 16384;

__global__ __launch_bounds__(kRouterThreads) void router_kernel(const float* __restrict__ x, int hidden,
                                                                const float* __restrict__ router, int n_experts,
                                                                int top_k, int norm, uint32_t* __restrict__ experts,
                                                                float* __restrict__ weights) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* xs = smem;             // [hidden]
  float* prob = smem + hidden;  // [n_experts + 1]: the logits, then their max
  double* ex = reinterpret_cast<double*>(smem + ((hidden + n_experts + 2) & ~1));  // [n_experts], 8-byte aligned
  const float* xr = x + (size_t)blockIdx.x * hidden;
  for (int i = threadIdx.x; i < hidden; i += kRouterThreads) xs[i] = xr[i];
  __syncthreads();
  for (int e = threadIdx.x; e < n_experts; e += kRouterThreads) {
    const float* w = router + (size_t)e * hidden;
    float acc = 0.f;
    for (int i = 0; i < hidden; ++i) acc += w[i] * xs[i];
    prob[e] = acc;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float mx = -INFINITY;
    for (int e = 0; e < n_experts; ++e)
      if (prob[e] > mx) mx = prob[e];
    prob[n_experts] = mx;  // the slot after the logits (the f64 array starts past it)
  }
  __syncthreads();
  const double m = (double)prob[n_experts];
  for (int e = threadIdx.x; e < n_experts; e += kRouterThreads) ex[e] = exp((double)prob[e] - m);
  __syncthreads();
  if (threadIdx.x != 0) return;
  double sum = 0.0;
  for (int e = 0; e < n_experts; ++e) sum += ex[e];
  const float inv = (float)(1.0 / sum);
  for (int e = 0; e < n_experts; ++e) prob[e] = (float)ex[e] * inv;
  uint32_t* eo = experts + (size_t)blockIdx.x * top_k;
  float* wo = weights + (size_t)blockIdx.x * top_k;
  for (int k = 0; k < top_k; ++k) {
    int best_e = 0;
    float best_p = -INFINITY;
    for (int e = 0; e < n_experts; ++e)
      if (prob[e] > best_p) {
        best_p = prob[e];
        best_e = e;
      }
    eo[k] = (uint32_t)best_e;
    wo[k] = best_p;
    prob[best_e] = -INFINITY;
  }
  if (norm) {
    float s = 0.f;
    for (int k = 0; k < top_k; ++k) s += wo[k];
    for (int k = 0; k < top_k; ++k) wo[k] = wo[k] / s;
  }
}

int32_t fail(rv_error* err, int32_t code, uint64_t a, uint64_t b, const char* what) {
  if (err) *err = rv_error{code, a, b, 0, 0, what};
  return code;
}

}  // namespace
}  // namespace rv

extern "C" int32_t rv_router_topk(const float* x, size_t n_rows, size_t hidden, const float* router,
                                  size_t router_len, size_t n_experts, size_t top_k, int norm_topk_prob,
                                  uint32_t* experts, float* weights, void* stream, uint32_t flags, rv_error* err) {
  using rv::fail;
  // forward.rs:774-777 validates top_k against the expert count first.
  if (top_k == 0 || top_k > n_experts) return fail(err, RV_FWD_INVALID_TOP_K, top_k, n_experts, "router top_k");
  if (hidden == 0) return fail(err, RV_PRIM_EMPTY, 0, 0, "router dot");
  size_t want;
  if (__builtin_mul_overflow(n_experts, hidden, &want) || want != router_len)
    return fail(err, RV_PRIM_LENGTH_MISMATCH, router_len, want, "router: weights vs n_experts x hidden");
  if (n_experts > (size_t)rv::kMaxExperts || hidden > (size_t)rv::kMaxHidden)
    return fail(err, RV_ERR_UNSUPPORTED, n_experts, hidden, "router above 1024 experts or 16384 values");
  if (flags & RV_HOST_PTRS) return fail(err, RV_ERR_UNSUPPORTED, flags, 0, "RV_HOST_PTRS (device pointers only)");
  const hipStream_t s = (hipStream_t)stream;
  if (n_rows > 0) {
    for (const void* p : {(const void*)x, (const void*)router, (const void*)experts, (const void*)weights})
      if (!p || ((uintptr_t)p & 3)) return fail(err, p ? RV_ERR_UNSUPPORTED : RV_ERR_NULL_ARG, (uintptr_t)p, 0, "router pointer");
    const size_t lds = ((hidden + n_experts + 2) & ~(size_t)1) * 4 + n_experts * 8;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&rv::router_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    hipLaunchKernelGGL(rv::router_kernel, dim3((unsigned)n_rows), dim3(rv::kRouterThreads), (unsigned)lds, s, x,
                       (int)hidden, router, (int)n_experts, (int)top_k, norm_topk_prob ? 1 : 0, experts, weights);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(err, RV_ERR_HIP, (uint64_t)e, 0, "router launch");
  }
  if (flags & RV_SYNC) {
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(err, RV_ERR_HIP, (uint64_t)e, 0, "hipStreamSynchronize");
  }
  if (err) *err = rv_error{RV_OK, 0, 0, 0, 0, nullptr};
  return RV_OK;
}
