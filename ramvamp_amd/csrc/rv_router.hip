// rv_router.hip — the MoE router's decision (include/ramvamp_router.h;
// model/forward.rs:2658-2705), bit for bit.
//
// One workgroup per row. Thread e computes expert e's logit as dot_f32 does
// (forward.rs:1231-1238): one serial f32 sum, each product rounded before it
// is added (contraction off), in index order. The row is staged in LDS; each
// thread streams its own expert's weight row with 16-byte loads, chunks
// ahead of the sum (rows 16-byte aligned; otherwise 4-byte loads in the
// same order), or, for 1 or 2 rows and at most 128 experts, the workgroup stages
// 64-value chunks of every row through LDS with coalesced loads (the staged
// form below). The softmax (softmax.rs:18-40) takes the max over
// the logits, each thread its exponential in f64, and one thread the f64 sum
// in expert order (the reference's order) and the f32 reciprocal. The top-k
// (strict >: the first index wins ties; the winner set to -inf) runs as a
// wave argmax that prefers the larger probability and then the lower index,
// which is the serial scan's choice; the renormalization is an f32 sum in
// selection order, then one division each.
#include <hip/hip_runtime.h>

#include "../../include/ramvamp_router.h"
#include "rv_device.hpp"
#include "rv_internal.hpp"

namespace rv {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxExperts = 1024;
constexpr int kMaxHidden = 16384;
constexpr int kChunk = 32;  // weight values per prefetched chunk

// Dynamic LDS per row: x [hidden], the logits [n_experts + 1], then the f64
// exponentials [n_experts]; rounded to 4 floats so every row's x starts
// 16-byte aligned for the chunked reads.
__host__ __device__ constexpr size_t router_lds_floats(size_t hidden, size_t n_experts) {
  return (((hidden + n_experts + 2) & ~(size_t)1) + 2 * n_experts + 3) & ~(size_t)3;
}

// The x values of chunk c for rows 0..R-1, read from LDS (row r's region
// starts row_stride floats after row r-1's).
template <int R>
__device__ __forceinline__ void load_x(f32x4 (&xv)[R][kChunk / 4], const float* __restrict__ xs, int row_stride,
                                       int c) {
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < kChunk / 4; ++q)
      xv[r][q] = *reinterpret_cast<const f32x4*>(xs + (size_t)r * row_stride + c * kChunk + 4 * q);
}

// acc[r] += w[j] * x_r[j] for one 32-value chunk of R rows, in order: the
// chunk's products first (independent, each rounded), then each row's
// dependent additions, so the sums' chains wait on additions only.
template <int R>
__device__ __forceinline__ void chunk_sum(float (&acc)[R], const f32x4 (&w)[kChunk / 4],
                                          const f32x4 (&xv)[R][kChunk / 4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float p[kChunk];
#pragma unroll
    for (int q = 0; q < kChunk / 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) p[4 * q + e] = w[q][e] * xv[r][q][e];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) acc[r] += p[k];
  }
}

// The staged form (1 or 2 rows per workgroup, at most 128 experts, hidden
// a multiple of 64, 16-byte aligned weights): the weight rows reach the sums
// through LDS in 64-value chunks. Each thread loads 8 of a chunk's 2048
// 16-byte quads (a wave: 4 experts' 16 consecutive quads each), three
// chunks ahead, and stores them into a 2-deep ring (rows padded to 68
// floats); lane e of waves 0 and 1 then sums expert e's chunk from LDS for
// each row, so no wave's load touches 64 scattered rows.
constexpr int kStagedChunk = 64;
constexpr int kStagedRow = kStagedChunk + 4;  // floats per staged expert row
constexpr int kStagedExperts = 128;
constexpr size_t kStagedBytes = 2 * kStagedExperts * kStagedRow * sizeof(float);

// R rows per workgroup (blockIdx.x * R ..), each with its LDS region of
// router_lds_floats(hidden, n_experts) floats; every weight chunk a thread
// loads feeds all R rows' sums. STAGED: the staged form above.
template <int R, bool STAGED>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(const float* __restrict__ x, int n_rows, int hidden,
                                                                const float* __restrict__ router, int n_experts,
                                                                int top_k, int norm, uint32_t* __restrict__ experts,
                                                                float* __restrict__ weights) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) float smem[];
  __shared__ __attribute__((aligned(16))) float wl[STAGED ? 2 * kStagedExperts * kStagedRow : 4];
  const int rs = (int)router_lds_floats(hidden, n_experts);  // floats per row region (a multiple of 4)
  const int row0 = (int)blockIdx.x * R, nr = min(R, n_rows - row0);
  auto xs_of = [&](int r) { return smem + (size_t)r * rs; };                 // [hidden]
  auto prob_of = [&](int r) { return smem + (size_t)r * rs + hidden; };      // [n_experts + 1]
  auto ex_of = [&](int r) {                                                  // [n_experts], 8-byte aligned
    return reinterpret_cast<double*>(smem + (size_t)r * rs + ((hidden + n_experts + 2) & ~1));
  };
  const int tid = threadIdx.x;
  for (int r = 0; r < R; ++r) {
    const float* xr = x + (size_t)(row0 + min(r, nr - 1)) * hidden;  // rows past the batch repeat its last
    for (int i = tid; i < hidden; i += kRouterThreads) xs_of(r)[i] = xr[i];
  }
  __syncthreads();
  if constexpr (STAGED) {
    const int nc = hidden / kStagedChunk;
    // Chunk c's quads of this thread (clamped to the last chunk, so every
    // prefetch is issued and the wait before a stash counts only newer
    // loads; experts past the last repeat it).
    auto fetch = [&](int c, f32x4 (&dst)[8]) {
      c = min(c, nc - 1);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int f = k * kRouterThreads + tid, e = min(f >> 4, n_experts - 1);
        dst[k] = *reinterpret_cast<const f32x4*>(router + (size_t)e * hidden + c * kStagedChunk + 4 * (f & 15));
      }
    };
    auto stash = [&](const f32x4 (&src)[8], int buf) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int f = k * kRouterThreads + tid;
        *reinterpret_cast<f32x4*>(&wl[(buf * kStagedExperts + (f >> 4)) * kStagedRow + 4 * (f & 15)]) = src[k];
      }
    };
    // Lanes 0..127, for each of the R rows: chunk c's rounded products, then
    // the row's serial additions (the rows' chains are independent).
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    auto sum_chunk = [&](int c, int buf) {
      if (tid >= kStagedExperts) return;  // waves 2 and 3 only stage
      const float* wr = &wl[(buf * kStagedExperts + tid) * kStagedRow];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float* xr = xs_of(r) + c * kStagedChunk;
        float p[kStagedChunk];
#pragma unroll
        for (int q = 0; q < kStagedChunk / 4; ++q) {
          const f32x4 w4 = *reinterpret_cast<const f32x4*>(wr + 4 * q), x4 = *reinterpret_cast<const f32x4*>(xr + 4 * q);
#pragma unroll
          for (int j = 0; j < 4; ++j) p[4 * q + j] = w4[j] * x4[j];
        }
#pragma unroll
        for (int k = 0; k < kStagedChunk; ++k) acc[r] += p[k];
      }
    };
    // Chunk j sits in ring slot j & 1 once staged; while the sums read chunk
    // c, chunk c + 1 is stashed into the other slot (read last in iteration
    // c - 1, before its barrier) and chunk c + 4 fetched into the registers
    // it leaves.
    f32x4 r0[8], r1[8], r2[8], r3[8];
    fetch(0, r0);
    fetch(1, r1);
    fetch(2, r2);
    fetch(3, r3);
    stash(r0, 0);
    fetch(4, r0);
    __syncthreads();
    int c = 0;
    for (; c + 4 <= nc; c += 4) {
      sum_chunk(c, 0);
      stash(r1, 1);
      fetch(c + 5, r1);
      __syncthreads();
      sum_chunk(c + 1, 1);
      stash(r2, 0);
      fetch(c + 6, r2);
      __syncthreads();
      sum_chunk(c + 2, 0);
      stash(r3, 1);
      fetch(c + 7, r3);
      __syncthreads();
      sum_chunk(c + 3, 1);
      stash(r0, 0);
      fetch(c + 8, r0);
      __syncthreads();
    }
    // Up to three chunks left: c in slot 0, c + 1 and c + 2 in r1 and r2.
    if (c < nc) {
      sum_chunk(c, 0);
      stash(r1, 1);
      __syncthreads();
    }
    if (c + 1 < nc) {
      sum_chunk(c + 1, 1);
      stash(r2, 0);
      __syncthreads();
    }
    if (c + 2 < nc) sum_chunk(c + 2, 0);
    if (tid < n_experts) {
#pragma unroll
      for (int r = 0; r < R; ++r) prob_of(r)[tid] = acc[r];
    }
  } else {
  const bool vec = hidden % 4 == 0 && ((uintptr_t)router & 15) == 0;
  const int nc = vec ? hidden / kChunk : 0;  // whole chunks; the rest one value at a time
  for (int g0 = 0; g0 < n_experts; g0 += kRouterThreads) {
    const int e = min(g0 + tid, n_experts - 1);
    const float* w = router + (size_t)e * hidden;
    const f32x4* wv = reinterpret_cast<const f32x4*>(w);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    // Chunk c of the weight row (clamped to the last: every prefetch is
    // issued, so the wait before each chunk's use counts only newer chunks'
    // loads), three ahead of its sums. Up to 2 rows, x is read from LDS one
    // chunk ahead too; 4 rows' worth would not fit the registers, so there
    // it is read just before its sums.
    constexpr bool x_ahead = R <= 2;
    auto fetch = [&](int c, f32x4 (&dst)[kChunk / 4]) {
      c = min(c, nc - 1);
#pragma unroll
      for (int q = 0; q < kChunk / 4; ++q) dst[q] = wv[c * (kChunk / 4) + q];
    };
    auto pre = [&](f32x4 (&xv)[R][kChunk / 4], int c) {
      if constexpr (x_ahead) load_x<R>(xv, smem, rs, c);
    };
    auto use = [&](const f32x4 (&wc)[kChunk / 4], f32x4 (&xv)[R][kChunk / 4], int c) {
      if constexpr (!x_ahead) load_x<R>(xv, smem, rs, c);
      chunk_sum<R>(acc, wc, xv);
    };
    if (nc > 0) {
      f32x4 r0[kChunk / 4], r1[kChunk / 4], r2[kChunk / 4], r3[kChunk / 4];
      f32x4 xa[R][kChunk / 4], xb[R][kChunk / 4];
      fetch(0, r0);
      fetch(1, r1);
      fetch(2, r2);
      pre(xa, 0);
      int c = 0;
      for (; c + 4 <= nc; c += 4) {
        fetch(c + 3, r3);
        pre(xb, c + 1);
        use(r0, xa, c);
        fetch(c + 4, r0);
        pre(xa, c + 2);
        use(r1, xb, c + 1);
        fetch(c + 5, r1);
        pre(xb, c + 3);
        use(r2, xa, c + 2);
        fetch(c + 6, r2);
        pre(xa, min(c + 4, nc - 1));
        use(r3, xb, c + 3);
      }
      // Up to three chunks left, already in r0, r1, r2 (x of the first in xa).
      if (c < nc) use(r0, xa, c);
      if (c + 1 < nc) {
        pre(xb, c + 1);
        use(r1, xb, c + 1);
      }
      if (c + 2 < nc) {
        pre(xa, c + 2);
        use(r2, xa, c + 2);
      }
    }
    for (int i = nc * kChunk; i < hidden; ++i) {
      const float wi = w[i];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += wi * xs_of(r)[i];
    }
    if (g0 + tid < n_experts) {
#pragma unroll
      for (int r = 0; r < R; ++r) prob_of(r)[g0 + tid] = acc[r];
    }
  }
  }
  __syncthreads();
  if (tid < nr) {  // thread r: row r's maximum
    const float* pr = prob_of(tid);
    float mx = -INFINITY;
    for (int e = 0; e < n_experts; ++e)
      if (pr[e] > mx) mx = pr[e];
    prob_of(tid)[n_experts] = mx;  // the slot after the logits (the f64 array starts past it)
  }
  __syncthreads();
  for (int r = 0; r < nr; ++r) {
    const double m = (double)prob_of(r)[n_experts];
    for (int e = tid; e < n_experts; e += kRouterThreads) ex_of(r)[e] = exp((double)prob_of(r)[e] - m);
  }
  __syncthreads();
  __shared__ float inv_sh[R];
  if (tid < nr) {  // thread r: row r's f64 sum in expert order
    const double* er = ex_of(tid);
    double sum = 0.0;
    for (int e = 0; e < n_experts; ++e) sum += er[e];
    inv_sh[tid] = (float)(1.0 / sum);
  }
  __syncthreads();
  for (int r = 0; r < nr; ++r) {
    const float inv = inv_sh[r];
    for (int e = tid; e < n_experts; e += kRouterThreads) prob_of(r)[e] = (float)ex_of(r)[e] * inv;
  }
  __syncthreads();
  // Wave r (< nr): row r's top_k rounds of an argmax, each lane over experts
  // lane, lane + 64, ... (in order, strict >), then across lanes preferring
  // the larger value and then the lower index; with nothing above -inf,
  // expert 0 at -inf.
  const int wave = tid >> 6, lane = tid & 63;
  if (wave >= nr) return;
  float* prob = prob_of(wave);
  uint32_t* eo = experts + (size_t)(row0 + wave) * top_k;
  float* wo = weights + (size_t)(row0 + wave) * top_k;
  float s = 0.f;
  for (int k = 0; k < top_k; ++k) {
    float bp = -INFINITY;
    int be = 1 << 30;
    for (int e = lane; e < n_experts; e += 64)
      if (prob[e] > bp) {
        bp = prob[e];
        be = e;
      }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float p2 = __shfl_xor(bp, off, 64);
      const int e2 = __shfl_xor(be, off, 64);
      if (p2 > bp || (p2 == bp && e2 < be)) {
        bp = p2;
        be = e2;
      }
    }
    if (be == (1 << 30)) be = 0;  // every probability -inf or NaN: the scan keeps expert 0
    if (lane == 0) {
      eo[k] = (uint32_t)be;
      wo[k] = bp;
      prob[be] = -INFINITY;
    }
    s += bp;  // the selection-order f32 sum, identical on every lane
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  }
  if (norm && lane == 0) {
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
    // Rows per workgroup: as many as keep at least 256 workgroups (up to 4)
    // and fit the LDS; each weight chunk a thread loads then feeds them all.
    const size_t row_bytes = rv::router_lds_floats(hidden, n_experts) * sizeof(float);
    const size_t lds_cap = 160 * 1024 - 1024;
    int R = 1;
    while (R < 4 && n_rows >= (size_t)(2 * R) * 256 && (size_t)(2 * R) * row_bytes <= lds_cap) R *= 2;
    const unsigned grid = (unsigned)((n_rows + R - 1) / R);
    // At most 128 experts and 1 or 2 rows per workgroup: the staged form
    // when the chunks divide the row and the ring fits beside the rows'
    // regions (4 rows staged measured slower: 72.4 vs 63.9 us for 1024 rows).
    const bool staged = R <= 2 && n_experts <= (size_t)rv::kStagedExperts && hidden % rv::kStagedChunk == 0 &&
                        ((uintptr_t)router & 15) == 0 && (size_t)R * row_bytes + rv::kStagedBytes <= lds_cap;
#define RV_ROUTER(RR, ST)                                                                                         \
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&rv::router_kernel<RR, ST>),                           \
                            hipFuncAttributeMaxDynamicSharedMemorySize,                                          \
                            (int)(ST ? lds_cap - rv::kStagedBytes : lds_cap));                                   \
  hipLaunchKernelGGL((rv::router_kernel<RR, ST>), dim3(grid), dim3(rv::kRouterThreads), (unsigned)(RR * row_bytes), \
                     s, x, (int)n_rows, (int)hidden, router, (int)n_experts, (int)top_k, norm_topk_prob ? 1 : 0,    \
                     experts, weights)
    if (R == 4) {
      RV_ROUTER(4, false);
    } else if (R == 2 && staged) {
      RV_ROUTER(2, true);
    } else if (R == 2) {
      RV_ROUTER(2, false);
    } else if (staged) {
      RV_ROUTER(1, true);
    } else {
      RV_ROUTER(1, false);
    }
#undef RV_ROUTER
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
