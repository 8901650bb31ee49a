/*
 * cast_bench.h - measurement aids of bench.py, built into libcast_bench.so
 * (not part of the product library libcast_amd.so).  No counterpart in the
 * reference.  Same conventions as cast_amd.h: device pointers, stream-ordered,
 * cast_status return codes.
 */
#ifndef CAST_BENCH_H
#define CAST_BENCH_H

#include <stdint.h>

#include "cast_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------
 * Measurement aid, no counterpart in the reference.  Samples the shader
 * clock: writes out[2*slot] = shader cycles and out[2*slot + 1] = ticks of
 * the constant 100 MHz counter over a fixed chain of `iters` dependent FMAs
 * (one workgroup, stream-ordered).  cycles / ticks * 100 MHz is the shader
 * clock at that point of the stream; bench.py uses it to separate a clock
 * ramp from a change in cycles per call.  out: uint64 [2 * (slot + 1)].
 * ------------------------------------------------------------------- */
int cast_clock_sample(uint64_t *out, int32_t slot, int32_t iters, cast_stream_t stream);

/* ---------------------------------------------------------------------
 * Measurement aid, no counterpart in the reference.  The MFMA ceiling at
 * the bf16 attention kernel's launch shape: `grid` workgroups of 512
 * threads at two waves per SIMD, each wave running `tiles` rounds of that
 * kernel's 32 v_mfma_f32_32x32x16_bf16 per 64-key tile (32768 FLOP each)
 * with no softmax and no global loads.  mode 0: operands in registers;
 * 1: every A operand read from LDS at the kernel's K / V^T addresses;
 * 3: those reads plus the per-tile workgroup barrier.
 *   src   bf16 operand values, src_chunks 16-byte chunks (read modulo)
 *   out   float [grid * 512]   the accumulator sums (keeps the work live)
 *   clk   uint64 [2 * grid]    per workgroup: shader cycles, 100 MHz ticks
 * bench.py uses it to state what the matrix pipes sustain on this part
 * next to the attention kernel's rate.
 * ------------------------------------------------------------------- */
int cast_mfma_ceiling(const void *src, int64_t src_chunks, float *out, uint64_t *clk, int32_t grid,
                      int32_t tiles, int32_t mode, cast_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CAST_BENCH_H */
