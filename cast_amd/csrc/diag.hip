// Measurement aid (no counterpart in the reference): samples the shader
// clock next to the constant 100 MHz clock, so that a benchmark can tell a
// change of clock frequency from a change of cycles per call.
#include "cast_common.hpp"

namespace cast {

// One thread times a fixed chain of dependent FMAs with the shader cycle
// counter (clock64) and the constant-rate counter (wall_clock64).
__global__ void clock_sample_kernel(uint64_t *out, int32_t slot, int32_t iters) {
    if (threadIdx.x != 0) return;
    const uint64_t c0 = clock64(), w0 = wall_clock64();
    float x = 1.0f;
    for (int i = 0; i < iters; ++i) x = __builtin_fmaf(x, 1.0000001f, 1e-7f);
    const uint64_t c1 = clock64(), w1 = wall_clock64();
    out[2 * slot] = c1 - c0;
    out[2 * slot + 1] = (w1 - w0) + (x == 12345.f ? 1u : 0u);   // keeps the chain live
}

}  // namespace cast

extern "C" int cast_clock_sample(uint64_t *out, int32_t slot, int32_t iters, cast_stream_t stream) {
    if (!out) return CAST_ERR_NULL_POINTER;
    if (slot < 0 || iters < 0) return CAST_ERR_SHAPE;
    cast::clock_sample_kernel<<<1, 64, 0, reinterpret_cast<hipStream_t>(stream)>>>(out, slot, iters);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}
