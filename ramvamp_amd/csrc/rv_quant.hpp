// rv_quant.hpp — launchers of the quantized-projection kernels (rv_quant.hip),
// called by the validating C ABI in rv_gemv_abi.cpp. Every launcher assumes
// its arguments were validated: lengths, formats and 4-byte alignment.
#pragma once

#include "../../include/ramvamp_gemv.h"
#include "rv_internal.hpp"

namespace rv {

// The fused projections (one launch): up to three row ranges of
// independent matrices, each against the Q8_K (k-quant formats) or the Q8_0
// (RV_QF_Q8_0) form of one f32 activation row x, which each workgroup
// quantizes into LDS before its rows run. x holds nbk * 256 = nb0 * 32
// values, at most kFusedMaxKBlocks * 256.
constexpr int kFusedWaves = 8;
constexpr int kFusedMaxKBlocks = 32;
constexpr int kFusedMax0Blocks = kFusedMaxKBlocks * 8;
struct FusedSeg {
  uint32_t fmt;
  const uint8_t* w;
  size_t row_bytes;
  float* out;
};
struct FusedProjArgs {
  const float* x;
  int nbk, nb0;
  int n_seg;
  FusedSeg seg[3];
  int n_rows[3];
};

HipStatus launch_quantize_q8_k(const float* x, rv_block_q8_k* out, size_t n_blocks, hipStream_t s);
HipStatus launch_quantize_q8_0(const float* x, rv_block_q8_0* out, size_t n_blocks, hipStream_t s);
// out[i] = row(row_lo + i) . acts, i < n_rows; acts quantized blocks
// (Q8_K, or Q8_0 for RV_QF_Q8_0) in global memory.
HipStatus launch_gemv_rows(uint32_t fmt, const uint8_t* w, size_t row_bytes, size_t in_dim, const void* acts,
                           size_t row_lo, size_t n_rows, float* out, hipStream_t s);
HipStatus launch_fused_proj(const FusedProjArgs& a, hipStream_t s);
// out[0 .. n) = 0 (a kernel, so the call can be captured into a graph).
HipStatus launch_fill_zero(float* out, size_t n, hipStream_t s);

}  // namespace rv
