// rv_device.hpp — device helpers shared by the gfx950 kernels.
//
// Wave64 only (CDNA4): every lane-group reduction below assumes 64-lane
// wavefronts and uses DPP row operations, which act within 16-lane rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// DPP controls (GFX9 encoding).
enum : int {
  DPP_QUAD_XOR1 = 0xB1,       // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,       // quad_perm [2,3,0,1]
  DPP_ROW_HALF_MIRROR = 0x141,
  DPP_ROW_MIRROR = 0x140,
};

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N = 2, 4, 8, 16, 32); every lane of a
// group ends with the group's total. Within 16 lanes this is four DPP steps
// (pairs, quads, half-row mirror, row mirror); 32 adds one cross-row swap.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32, "group size");
  x += dpp_f32<DPP_QUAD_XOR1>(x);
  if constexpr (N >= 4) x += dpp_f32<DPP_QUAD_XOR2>(x);
  if constexpr (N >= 8) x += dpp_f32<DPP_ROW_HALF_MIRROR>(x);
  if constexpr (N >= 16) x += dpp_f32<DPP_ROW_MIRROR>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16, 64);
  return x;
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
  x = fmaxf(x, dpp_f32<DPP_QUAD_XOR1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp_f32<DPP_QUAD_XOR2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp_f32<DPP_ROW_HALF_MIRROR>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp_f32<DPP_ROW_MIRROR>(x));
  if constexpr (N >= 32) x = fmaxf(x, __shfl_xor(x, 16, 64));
  return x;
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double x) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(x), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(x), CTRL, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}

// x + (x of the lane 16 or 32 apart): a permlane swap pairs every lane with
// that partner, and the pair's two values are summed (the same sum on both
// lanes, addition being commutative).
template <int D>
__device__ __forceinline__ double swap_sum_f64(double x) {
  const unsigned lo = (unsigned)__double2loint(x), hi = (unsigned)__double2hiint(x);
  if constexpr (D == 16) {
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return __hiloint2double((int)h[0], (int)l[0]) + __hiloint2double((int)h[1], (int)l[1]);
  } else {
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return __hiloint2double((int)h[0], (int)l[0]) + __hiloint2double((int)h[1], (int)l[1]);
  }
}

// max(x, x of the lane 16 or 32 apart), on every lane, by a permlane swap
// (VALU; no LDS round trip as a bpermute shuffle would take).
template <int D>
__device__ __forceinline__ float swap_max(float x) {
  const unsigned u = __float_as_uint(x);
  if constexpr (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
}

// x + (x of the lane 16 or 32 apart), on every lane (the same sum on both
// lanes of a pair).
template <int D>
__device__ __forceinline__ float swap_sum(float x) {
  const unsigned u = __float_as_uint(x);
  if constexpr (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Wave total in f64 on every lane: DPP within 16-lane rows, then the two
// cross-row swaps (all VALU, no LDS round trips).
__device__ __forceinline__ double wave_sum_f64(double x) {
  x += dpp_f64<DPP_QUAD_XOR1>(x);
  x += dpp_f64<DPP_QUAD_XOR2>(x);
  x += dpp_f64<DPP_ROW_HALF_MIRROR>(x);
  x += dpp_f64<DPP_ROW_MIRROR>(x);
  x = swap_sum_f64<16>(x);
  return swap_sum_f64<32>(x);
}

// f32 -> f16 bits, round to nearest even, with the reference's subnormal,
// overflow and NaN encodings (crates/core/src/kernels/quants/f16.rs:39-91).
// Integer-only, so the result never depends on the hardware rounding mode or
// its NaN quieting.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  uint32_t bits = __float_as_uint(x);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exp = (int32_t)((bits >> 23) & 0xFF);
  uint32_t frac = bits & 0x007FFFFFu;
  if (exp == 0xFF) return (uint16_t)(frac == 0 ? (sign | 0x7C00u) : (sign | 0x7E00u | ((frac >> 13) & 0x03FFu)));
  int32_t e16 = exp - 112;
  if (e16 >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e16 <= 0) {
    if (e16 < -10) return (uint16_t)sign;
    uint32_t mant = exp == 0 ? frac : (frac | 0x00800000u);
    uint32_t shift = (uint32_t)(14 - e16);
    uint32_t ulp = 1u << shift, half = ulp >> 1;
    uint32_t v = mant >> shift, rem = mant & (ulp - 1);
    if (rem > half || (rem == half && (v & 1u))) v += 1;
    return (uint16_t)(sign | v);
  }
  uint32_t v = ((uint32_t)e16 << 10) | (frac >> 13);
  uint32_t rem = frac & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v += 1;
  return (uint16_t)(sign | v);
}

// Eight consecutive plane elements widened to f32 (f16 widening is exact).
__device__ __forceinline__ void load8(const float* __restrict__ p, float (&x)[8]) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
  x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
}
__device__ __forceinline__ void load8(const _Float16* __restrict__ p, float (&x)[8]) {
  f16x8 h = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)h[i];
}

// 16 bytes per lane from global memory straight into LDS at the wave-uniform
// base `l` + 16 * lane (global_load_lds_dwordx4). The device-only guard keeps
// the host pass, which has no such builtin, from dropping the kernels' stubs.
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void lds_load16(const void* g, lds_void* l) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
#endif
}

// The same copy issued from inline assembly, to the LDS byte offset `l`: the
// compiler does not see it write LDS, so it adds no wait for it before later
// LDS reads (for the builtin it waits for every outstanding load before any
// LDS read whose address it cannot tell apart, which serialises a ring of
// stages indexed at run time). The caller orders every read of the
// destination after the copy itself: wait_vmcnt, then a barrier when other
// waves read it. m0 is an input operand, so the compiler loads it; the
// s_nop covers the one wait state between an m0 write and an LDS DMA.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t l) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(l) : "memory");
#endif
}
__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)p; }
// The same copy with a wave-uniform base in scalar registers and the lane's
// byte offset in a vector register (no per-copy 64-bit vector add).
__device__ __forceinline__ void lds_dma16s(const void* sbase, uint32_t voff, uint32_t l) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(l) : "memory");
}

// s_waitcnt with vmcnt(n) and the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace rv
