// Helpers shared by the streamed rollout kernels: LDS accesses by byte offset, bf16 packing on
// gfx950's conversion instruction, packed bf16 ReLU.
#pragma once

#include <type_traits>

#include "nca_rollout.h"

namespace nca {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

inline unsigned st_al16(unsigned v) { return (v + 15u) & ~15u; }

__device__ __forceinline__ uint2 lds_ld64(const unsigned char *s, unsigned off) {
    return *reinterpret_cast<const uint2 *>(s + off);
}
__device__ __forceinline__ float4 lds_ld128f(const unsigned char *s, unsigned off) {
    return *reinterpret_cast<const float4 *>(s + off);
}
__device__ __forceinline__ void lds_st64(unsigned char *s, unsigned off, uint2 v) {
    *reinterpret_cast<uint2 *>(s + off) = v;
}
__device__ __forceinline__ void lds_st128(unsigned char *s, unsigned off, uint4 v) {
    *reinterpret_cast<uint4 *>(s + off) = v;
}
__device__ __forceinline__ void lds_st128f(unsigned char *s, unsigned off, float4 v) {
    *reinterpret_cast<float4 *>(s + off) = v;
}
typedef float f32x2 __attribute__((ext_vector_type(2)));
// two floats to packed bf16 (round to nearest even): one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    const f32x2 f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}
// ReLU of two packed bf16 values: a negative bf16 is a negative int16.
__device__ __forceinline__ uint32_t relu_bf16x2(uint32_t v) {
    const s16x2 x = __builtin_bit_cast(s16x2, v);
    const s16x2 z = {0, 0};
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(x, z));
}
__device__ __forceinline__ short bf16_bits(float v) { return __builtin_bit_cast(short, (__bf16)v); }

}  // namespace nca
