// rv_quant.hpp — launchers of the quantized-projection kernels (rv_quant.hip),
// called by the validating C ABI in rv_gemv_abi.cpp. Every launcher assumes
// its arguments were validated: lengths, formats and 4-byte alignment.
#pragma once

#include "../../include/ramvamp_gemv.h"
#include "rv_internal.hpp"

namespace rv {

// One segment of the fused attention-input projection: n rows of a weight
// matrix against one activation row (Q8_K blocks, or Q8_0 for RV_QF_Q8_0).
struct InProjSeg {
  uint32_t fmt;
  const uint8_t* w;
  size_t row_bytes;
  int nb;  // blocks per row
  const void* acts;
  float* out;
};
struct InProjArgs {
  InProjSeg seg[3];  // q, k, v
  int n_rows[3];
};

HipStatus launch_quantize_q8_k(const float* x, rv_block_q8_k* out, size_t n_blocks, hipStream_t s);
HipStatus launch_quantize_q8_0(const float* x, rv_block_q8_0* out, size_t n_blocks, hipStream_t s);
// out[i] = row(row_lo + i) . acts, i < n_rows.
HipStatus launch_gemv_rows(uint32_t fmt, const uint8_t* w, size_t row_bytes, size_t in_dim, const void* acts,
                           size_t row_lo, size_t n_rows, float* out, hipStream_t s);
HipStatus launch_in_proj(const InProjArgs& a, hipStream_t s);
// out[0 .. n) = 0 (a kernel, so the call can be captured into a graph).
HipStatus launch_fill_zero(float* out, size_t n, hipStream_t s);

}  // namespace rv
