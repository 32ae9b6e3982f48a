// Device-side helpers shared by the gfx950 kernels of libhmx: bf16 bit
// conversions, 16-byte vector access, wave64 reductions and the fused
// epilogue activations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hmx_internal.hpp"

namespace hmx {

constexpr int kWave = 64;

// bf16 is carried as its raw 16 bits; arithmetic is always f32.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Round-to-nearest-even f32 -> bf16, NaN kept quiet (the rounding torch's
// `.to(torch.bfloat16)` performs).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// Element access by storage type: float or bf16 (uint16_t bits).
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kPerVec = 4;  // elements per 16-byte vector
  __device__ static __forceinline__ float load(const float* p) { return *p; }
  __device__ static __forceinline__ void store(float* p, float v) { *p = v; }
  __device__ static __forceinline__ void unpack(const uint4& v, float* out) {
    out[0] = __uint_as_float(v.x);
    out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z);
    out[3] = __uint_as_float(v.w);
  }
  __device__ static __forceinline__ uint4 pack(const float* in) {
    return make_uint4(__float_as_uint(in[0]), __float_as_uint(in[1]),
                      __float_as_uint(in[2]), __float_as_uint(in[3]));
  }
};
template <> struct Elem<uint16_t> {
  static constexpr int kPerVec = 8;
  __device__ static __forceinline__ float load(const uint16_t* p) {
    return bf16_bits_to_f32(*p);
  }
  __device__ static __forceinline__ void store(uint16_t* p, float v) {
    *p = (uint16_t)f32_to_bf16_bits(v);
  }
  __device__ static __forceinline__ void unpack(const uint4& v, float* out) {
    out[0] = __uint_as_float(v.x << 16);
    out[1] = __uint_as_float(v.x & 0xffff0000u);
    out[2] = __uint_as_float(v.y << 16);
    out[3] = __uint_as_float(v.y & 0xffff0000u);
    out[4] = __uint_as_float(v.z << 16);
    out[5] = __uint_as_float(v.z & 0xffff0000u);
    out[6] = __uint_as_float(v.w << 16);
    out[7] = __uint_as_float(v.w & 0xffff0000u);
  }
  __device__ static __forceinline__ uint4 pack(const float* in) {
    return make_uint4(pack_bf16x2(in[0], in[1]), pack_bf16x2(in[2], in[3]),
                      pack_bf16x2(in[4], in[5]), pack_bf16x2(in[6], in[7]));
  }
};

// Load an f32 value of a vector operand whose storage dtype is a runtime code.
__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t i) {
  return dtype == HMX_DTYPE_BF16 ? bf16_bits_to_f32(((const uint16_t*)p)[i])
                                 : ((const float*)p)[i];
}

// Wave64 reductions: xor butterflies over all 64 lanes, every lane ends with
// the result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// exp through the hardware base-2 exponential.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// The activations a fused epilogue may apply to an f32 value, codes as in
// `hmx_epilogue`. `arg` is LeakyReLU's negative slope.
__device__ __forceinline__ float apply_activation(int code, float x, float arg) {
  switch (code) {
    case HMX_EPI_RELU:
      return x > 0.f ? x : (x != x ? x : 0.f);
    case HMX_EPI_SILU:
      return x / (1.f + __expf(-x));
    case HMX_EPI_SIGMOID:
      return 1.f / (1.f + __expf(-x));
    case HMX_EPI_GELU:
      return 0.5f * x * (1.f + erff(x * 0.7071067811865476f));
    case HMX_EPI_GELU_TANH: {
      const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      return 0.5f * x * (1.f + tanhf(u));
    }
    case HMX_EPI_TANH:
      return tanhf(x);
    case HMX_EPI_LEAKY_RELU:
      return x >= 0.f ? x : x * arg;
    default:
      return x;
  }
}

}  // namespace hmx
