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

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16 (lo in bits 0-15) with one v_cvt_pk_bf16_f32:
// round to nearest even, NaN kept NaN -- the rounding of torch's
// `.to(torch.bfloat16)`.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return pack_bf16x2(f, 0.f) & 0xffffu;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte store with the non-temporal (streaming) hint. Streaming kernels
// write each output once and never read it back: with the hint the writes
// reach HBM without allocating cache lines, which measures ~25% more write
// bandwidth than plain stores on gfx950.
__device__ __forceinline__ void store16_stream(void* p, const uint4& v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, (u32x4_t*)p);
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

constexpr float kLog2e = 1.4426950408889634f;

// exp(x - m): the difference first, as exp(x - row_max) is written, then one
// v_exp_f32 of its base-2 scaling. Folding m into an FMA, exp2(x * log2e -
// m * log2e), would carry the rounding error of m * log2e (half an ulp of
// |m| * 1.44, over 128 once |m| passes ~3e9) into every exponent of the row:
// finite rows such as [1e10, 0] would overflow to inf / NaN.
__device__ __forceinline__ float exp_sub(float x, float m) {
  return __builtin_amdgcn_exp2f((x - m) * kLog2e);
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

// max / min that return NaN when either operand is NaN (torch.maximum /
// torch.minimum / clamp), unlike fmaxf / fminf.
__device__ __forceinline__ float max_nan(float a, float b) {
  return (a != a || b != b) ? a + b : fmaxf(a, b);
}
__device__ __forceinline__ float min_nan(float a, float b) {
  return (a != a || b != b) ? a + b : fminf(a, b);
}

// One instruction of an epilogue program (hmx_program): the f32 result of
// op on registers a, b and the constants. The formulas are the ones torch
// evaluates for the same operation on f32 tensors.
__device__ __forceinline__ float program_op(int op, float a, float b, float c0, float c1) {
  switch (op) {
    case HMX_OP_COPY: return a;
    case HMX_OP_NEG: return -a;
    case HMX_OP_ABS: return fabsf(a);
    case HMX_OP_RELU: return a > 0.f ? a : (a != a ? a : 0.f);
    case HMX_OP_SIGMOID: return 1.f / (1.f + expf(-a));
    case HMX_OP_TANH: return tanhf(a);
    case HMX_OP_SILU: return a / (1.f + expf(-a));
    case HMX_OP_GELU: return a * 0.5f * (1.f + erff(a * 0.7071067811865476f));
    case HMX_OP_GELU_TANH: {
      const float inner = 0.7978845608028654f * (a + 0.044715f * a * a * a);
      return 0.5f * a * (1.f + tanhf(inner));
    }
    case HMX_OP_EXP: return expf(a);
    case HMX_OP_LOG: return logf(a);
    case HMX_OP_SQRT: return sqrtf(a);
    case HMX_OP_RSQRT: return 1.f / sqrtf(a);
    case HMX_OP_RECIP: return 1.f / a;
    case HMX_OP_ERF: return erff(a);
    case HMX_OP_SIN: return sinf(a);
    case HMX_OP_COS: return cosf(a);
    case HMX_OP_LOG1P: return log1pf(a);
    case HMX_OP_EXPM1: return expm1f(a);
    case HMX_OP_FLOOR: return floorf(a);
    case HMX_OP_CEIL: return ceilf(a);
    case HMX_OP_TRUNC: return truncf(a);
    case HMX_OP_ROUND: return rintf(a);
    case HMX_OP_SOFTPLUS: return a * c0 > c1 ? a : log1pf(expf(a * c0)) / c0;
    case HMX_OP_MISH: return a * tanhf(log1pf(expf(a)));
    case HMX_OP_HARDSWISH: return a * min_nan(max_nan(a + 3.f, 0.f), 6.f) / 6.f;
    case HMX_OP_HARDSIGMOID: return min_nan(max_nan(a + 3.f, 0.f), 6.f) / 6.f;
    case HMX_OP_ELU: return a <= 0.f ? expm1f(a) * (c0 * c1) : a * c1;
    case HMX_OP_LEAKY_RELU: return a > 0.f ? a : a * c0;
    case HMX_OP_CLAMP: return min_nan(max_nan(a, c0), c1);
    case HMX_OP_ADD_C: return a + c0;
    case HMX_OP_MUL_C: return a * c0;
    case HMX_OP_DIV_C: return a / c0;
    case HMX_OP_RSUB_C: return c0 - a;
    case HMX_OP_RDIV_C: return c0 / a;
    case HMX_OP_POW_C: return powf(a, c0);
    case HMX_OP_ADD: return a + b;
    case HMX_OP_SUB: return a - b;
    case HMX_OP_MUL: return a * b;
    case HMX_OP_DIV: return a / b;
    case HMX_OP_MAX: return max_nan(a, b);
    case HMX_OP_MIN: return min_nan(a, b);
    case HMX_OP_POW: return powf(a, b);
    default: return a;
  }
}

// Register i of a program's register file. The index is uniform across the
// wave (it comes from the program), so a chain of selects reads it without
// dynamic indexing of private memory.
__device__ __forceinline__ float program_reg(const float (&r)[HMX_PROGRAM_REGS], int i) {
  float v = r[0];
#pragma unroll
  for (int j = 1; j < HMX_PROGRAM_REGS; ++j) v = i == j ? r[j] : v;
  return v;
}

// Runs program `p` on the value x (register 0) and extra (register 1).
__device__ __forceinline__ float run_program(const hmx_program& p, float x, float extra) {
  float r[HMX_PROGRAM_REGS];
  r[0] = x;
  r[1] = extra;
#pragma unroll
  for (int j = 2; j < HMX_PROGRAM_REGS; ++j) r[j] = 0.f;
#pragma unroll 1
  for (int i = 0; i < p.count; ++i) {
    const hmx_instr ins = p.code[i];
    const float y = program_op(ins.op, program_reg(r, ins.a), program_reg(r, ins.b), ins.c0, ins.c1);
#pragma unroll
    for (int j = 0; j < HMX_PROGRAM_REGS; ++j) r[j] = ins.dst == j ? y : r[j];
  }
  return program_reg(r, p.result);
}

// Applies the epilogue (activation code or program) to n values in place,
// one value per pass of a loop that is not unrolled: the values rotate
// through v[0], so the program's code is emitted once however large n is.
template <int N>
__device__ __forceinline__ void run_program_n(const hmx_program& p, float (&v)[N], const float (&extra)[N]) {
  float e[N];
#pragma unroll
  for (int i = 0; i < N; ++i) e[i] = extra[i];
#pragma unroll 1
  for (int t = 0; t < N; ++t) {
    const float y = run_program(p, v[0], e[0]);
#pragma unroll
    for (int i = 0; i + 1 < N; ++i) {
      v[i] = v[i + 1];
      e[i] = e[i + 1];
    }
    v[N - 1] = y;
    e[N - 1] = 0.f;
  }
}

}  // namespace hmx
