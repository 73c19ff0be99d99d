// Shared device helpers for the gfx950 kernels of libglm53_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "glm53.h"

namespace glm53 {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define GLM53_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Pack two fp32 into a dword of two bf16 (lo in bits 0..15), RNE.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// Wave-uniform value in a scalar register.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    uint32_t other = (uint32_t)__shfl_xor((int)v, o, 64);
    v = v > other ? v : other;
  }
  return v;
}

}  // namespace glm53
