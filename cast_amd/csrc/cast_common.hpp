// Shared device helpers for the gfx950 tree-verification kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cast_amd.h"

namespace cast {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxPack = 128;      // two 64-bit ancestor words per row
constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_float(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

// Round-to-nearest-even float -> bf16 pair (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 p = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ void raise_flag(int32_t *status, int32_t bit) {
    if (status) atomicOr(status, bit);
}

// The value held by lane (l ^ 32).
__device__ __forceinline__ float partner32(float x) { return __shfl_xor(x, 32); }

}  // namespace cast
