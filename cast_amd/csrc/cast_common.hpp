// Shared device helpers for the gfx950 tree-verification kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cast_amd.h"

namespace cast {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
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

// Round-to-nearest-even float -> IEEE half pair (v_cvt_pk_f16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    f16x2 p = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ float f16_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// The two 16-bit element formats of the MFMA attention kernels: the 8-wide
// operand of v_mfma_f32_32x32x16_{bf16,f16}, that product, the rounding of
// a float pair to the format and the widening of one element.
struct Bf16 {
    using vec8 = bf16x8;
    static __device__ __forceinline__ floatx16 mma(vec8 a, vec8 b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
    static __device__ __forceinline__ float widen(uint16_t h) { return bf16_to_float(h); }
};
struct Fp16 {
    using vec8 = f16x8;
    static __device__ __forceinline__ floatx16 mma(vec8 a, vec8 b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_f16x2(lo, hi); }
    static __device__ __forceinline__ float widen(uint16_t h) { return f16_to_float(h); }
};

__device__ __forceinline__ void raise_flag(int32_t *status, int32_t bit) {
    if (status) atomicOr(status, bit);
}

// The value held by lane (l ^ 32).
__device__ __forceinline__ float partner32(float x) { return __shfl_xor(x, 32); }

}  // namespace cast
