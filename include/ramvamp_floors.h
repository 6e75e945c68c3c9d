/*
 * ramvamp_floors.h — measurement floors (no reference counterpart).
 *
 * Four probe launches that bench.py times (`--floors`, and `extra.floors`
 * in its default run) to measure the limits the attention kernels are judged
 * against on the box they run on: the cost of a launch in a graph, a plain
 * streaming read of a decode call's bytes, the issue rate of the MFMA forms
 * the kernels use, and how much VALU work an MFMA hides. They compute
 * nothing the library needs.
 *
 * Device pointers; work on `stream` (a hipStream_t, null for the null
 * stream).
 */
#ifndef RAMVAMP_FLOORS_H
#define RAMVAMP_FLOORS_H

#include <stddef.h>
#include <stdint.h>

#include "ramvamp_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One launch of a kernel of one 64-thread workgroup that does nothing. */
int32_t rv_floor_empty(void* stream, rv_error* err);

/* A streaming read of `bytes` (a multiple of 16) at src (16-byte aligned) by
 * n_wg workgroups of 256 threads: workgroup b reads the b-th contiguous
 * share with 16-byte non-temporal loads, eight in flight per thread, and
 * writes one float (the sum of its share, so nothing is optimised away) to
 * sink[b]. n_wg in [1, 65536]. */
int32_t rv_floor_stream_read(const void* src, size_t bytes, uint32_t n_wg, float* sink, void* stream, rv_error* err);

/* MFMA issue rate: n_wg workgroups of 256 threads, every wave issuing
 * `iters` rounds of `chains` independent accumulator chains of one form:
 * RV_FLOOR_MFMA_F16_16X16X32 (v_mfma_f32_16x16x32_f16, 16,384 FLOP),
 * RV_FLOOR_MFMA_F16_32X32X16 (v_mfma_f32_32x32x16_f16, 32,768 FLOP),
 * RV_FLOOR_MFMA_F32_16X16X4 (v_mfma_f32_16x16x4_f32, 2,048 FLOP). Each wave
 * writes one float to sink[wave]. chains: 1, 2 or 4; iters >= 1;
 * n_wg in [1, 65536]. The FLOPs are n_wg * 4 * iters * chains * the form's. */
#define RV_FLOOR_MFMA_F16_16X16X32 0
#define RV_FLOOR_MFMA_F16_32X32X16 1
#define RV_FLOOR_MFMA_F32_16X16X4 2
int32_t rv_floor_mfma(int32_t form, uint32_t chains, uint32_t iters, uint32_t n_wg, float* sink, void* stream,
                      rv_error* err);

/* MFMA / VALU overlap: n_wg workgroups of 256 threads, every wave issuing
 * `iters` rounds of 4 independent v_mfma_f32_32x32x16_f16 chains, each MFMA
 * followed in issue order by `valu_per_mfma` (0, 2, 4 or 8) independent VALU
 * instructions of one kind: RV_FLOOR_VALU_FMA (v_fma_f32) or
 * RV_FLOOR_VALU_EXP (v_exp_f32). The time per MFMA against valu_per_mfma = 0
 * shows how much VALU work an MFMA hides on the same SIMD. Each wave writes
 * one float to sink[wave]. iters >= 1; n_wg in [1, 65536]. */
#define RV_FLOOR_VALU_FMA 0
#define RV_FLOOR_VALU_EXP 1
int32_t rv_floor_mfma_valu(int32_t kind, uint32_t valu_per_mfma, uint32_t iters, uint32_t n_wg, float* sink,
                           void* stream, rv_error* err);

#ifdef __cplusplus
}
#endif

#endif /* RAMVAMP_FLOORS_H */
