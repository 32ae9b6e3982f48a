// Device-side helpers shared by the gfx950 kernels of libhmx: bf16 bit
// conversions, 16-byte vector access, wave64 reductions and the fused
// epilogue activations.
#pragma once

#ifdef __HIPCC_RTC__
// Run-time compilation (hipRTC, hmx_jit.cpp): no host headers; the
// fixed-width integer types live in __hip_internal.
using __hip_internal::int16_t;
using __hip_internal::int32_t;
using __hip_internal::int64_t;
using __hip_internal::int8_t;
using __hip_internal::uint16_t;
using __hip_internal::uint32_t;
using __hip_internal::uint64_t;
using __hip_internal::uint8_t;
typedef __hip_internal::uint64_t uintptr_t;
#include "hmx.h"
#else
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hmx_internal.hpp"
#endif

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

// A 16-byte store written through to memory (the system-scope coherence bits
// of a vector store), for outputs a kernel's last instructions write: the
// release at the kernel's end then has fewer dirty L2 lines to write back.
// A vector store of more than 8 bytes reads its data registers after issue,
// and the compiler does not see this store: the s_nop keeps the next
// instructions from overwriting them first.
__device__ __forceinline__ void store16_through(void* p, const uint4& v) {
  const u32x4_t d = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1" ::"v"(p), "v"(d) : "memory");
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
    // SiLU and sigmoid divide by 1 + e^-x with v_rcp_f32 (1 ulp) rather than
    // the correctly rounded division (~10 instructions more per value): in a
    // GEMM epilogue the division alone cost ~5 % of config 4's time. Both
    // keep torch's limits: -0 for x -> -inf's finite side, x for large x,
    // NaN for -inf and NaN.
    case HMX_EPI_SILU:
      return x * __builtin_amdgcn_rcpf(1.f + __expf(-x));
    case HMX_EPI_SIGMOID:
      return __builtin_amdgcn_rcpf(1.f + __expf(-x));
    case HMX_EPI_GELU: {
      // 0.5 x (1 + erf(x / sqrt 2)) with erfc(z), z = |x| / sqrt 2, by
      // Abramowitz & Stegun 7.1.26 (|error of erf| <= 1.5e-7): one
      // reciprocal, a degree-5 polynomial and one exponential, the same
      // instructions for every lane (the library erff branches on |z| < 1,
      // and a GEMM epilogue of it cost a third of config 4's time).
      // 1 + erf(x / sqrt 2) is 2 - erfc(z) for x >= 0, erfc(z) below (no
      // cancellation), but the formula's error bound is absolute: on the
      // negative side, where GELU is small, the relative error grows (about
      // 3e-6 at x = -2, 1.6e-3 at x = -5, 4e-2 at x = -13).
      const float z = fabsf(x) * 0.7071067811865476f;
      const float t = __builtin_amdgcn_rcpf(1.f + 0.3275911f * z);
      const float poly =
          t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
      const float erfc_z = poly * __expf(-z * z);
      return 0.5f * x * (x >= 0.f ? 2.f - erfc_z : erfc_z);
    }
    case HMX_EPI_GELU_TANH: {
      // 0.5 x (1 + tanh(u)) = x / (1 + e^(-2u)) exactly: one exponential and
      // a reciprocal instead of tanhf, with the same limits (x for u -> inf,
      // -0 for u -> -inf, NaN for NaN).
      const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      return x * __builtin_amdgcn_rcpf(1.f + __expf(-2.f * u));
    }
    case HMX_EPI_TANH: {
      // tanh x = sign(x) (1 - 2 / (1 + e^(2|x|))) from |x| = 0.25 on, the
      // odd Taylor series to x^9 below it (truncation under 1e-8 relative):
      // one exponential and a reciprocal, no branch across lanes, within
      // ~7 ulps of tanh (the library tanhf cost a GEMM epilogue ~9 % of
      // config 4). Limits: ±1 at ±inf, -0 at -0, NaN at NaN.
      const float a = fabsf(x);
      const float big = 1.f - 2.f * __builtin_amdgcn_rcpf(1.f + __expf(2.f * a));
      const float x2 = x * x;
      const float small =
          x * (1.f + x2 * (-0.33333334f + x2 * (0.13333334f + x2 * (-0.053968254f + x2 * 0.021869488f))));
      return a < 0.25f ? small : copysignf(big, x);
    }
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

// The operations of an epilogue program (hmx_program): X(opcode, f32 result of
// a, b and the constants c0, c1). The formulas are the ones torch evaluates
// for the same operation on f32 tensors, except the activations that also
// have a named code (sigmoid, tanh, SiLU, GELU and its tanh form), which take
// that code's form (apply_activation): a program's SiLU is the named SiLU.
#define HMX_PROGRAM_OPS(X)                                                       \
  X(HMX_OP_COPY, a)                                                              \
  X(HMX_OP_NEG, -a)                                                              \
  X(HMX_OP_ABS, fabsf(a))                                                        \
  X(HMX_OP_RELU, a > 0.f ? a : (a != a ? a : 0.f))                               \
  X(HMX_OP_SIGMOID, apply_activation(HMX_EPI_SIGMOID, a, 0.f))                   \
  X(HMX_OP_TANH, apply_activation(HMX_EPI_TANH, a, 0.f))                         \
  X(HMX_OP_SILU, apply_activation(HMX_EPI_SILU, a, 0.f))                         \
  X(HMX_OP_GELU, apply_activation(HMX_EPI_GELU, a, 0.f))                         \
  X(HMX_OP_GELU_TANH, apply_activation(HMX_EPI_GELU_TANH, a, 0.f))               \
  X(HMX_OP_EXP, expf(a))                                                         \
  X(HMX_OP_LOG, logf(a))                                                         \
  X(HMX_OP_SQRT, sqrtf(a))                                                       \
  X(HMX_OP_RSQRT, 1.f / sqrtf(a))                                                \
  X(HMX_OP_RECIP, 1.f / a)                                                       \
  X(HMX_OP_ERF, erff(a))                                                         \
  X(HMX_OP_SIN, sinf(a))                                                         \
  X(HMX_OP_COS, cosf(a))                                                         \
  X(HMX_OP_LOG1P, log1pf(a))                                                     \
  X(HMX_OP_EXPM1, expm1f(a))                                                     \
  X(HMX_OP_FLOOR, floorf(a))                                                     \
  X(HMX_OP_CEIL, ceilf(a))                                                       \
  X(HMX_OP_TRUNC, truncf(a))                                                     \
  X(HMX_OP_ROUND, rintf(a))                                                      \
  X(HMX_OP_SOFTPLUS, a * c0 > c1 ? a : log1pf(expf(a * c0)) / c0)                \
  X(HMX_OP_MISH, a * tanhf(log1pf(expf(a))))                                     \
  X(HMX_OP_HARDSWISH, a * min_nan(max_nan(a + 3.f, 0.f), 6.f) / 6.f)             \
  X(HMX_OP_HARDSIGMOID, min_nan(max_nan(a + 3.f, 0.f), 6.f) / 6.f)               \
  X(HMX_OP_ELU, a <= 0.f ? expm1f(a) * (c0 * c1) : a * c1)                       \
  X(HMX_OP_LEAKY_RELU, a > 0.f ? a : a * c0)                                     \
  X(HMX_OP_CLAMP, min_nan(max_nan(a, c0), c1))                                   \
  X(HMX_OP_ADD_C, a + c0)                                                        \
  X(HMX_OP_MUL_C, a * c0)                                                        \
  X(HMX_OP_DIV_C, a / c0)                                                        \
  X(HMX_OP_RSUB_C, c0 - a)                                                       \
  X(HMX_OP_RDIV_C, c0 / a)                                                       \
  X(HMX_OP_POW_C, powf(a, c0))                                                   \
  X(HMX_OP_ADD, a + b)                                                           \
  X(HMX_OP_SUB, a - b)                                                           \
  X(HMX_OP_MUL, a * b)                                                           \
  X(HMX_OP_DIV, a / b)                                                           \
  X(HMX_OP_MAX, max_nan(a, b))                                                   \
  X(HMX_OP_MIN, min_nan(a, b))                                                   \
  X(HMX_OP_POW, powf(a, b))

// One instruction on one value.
__device__ __forceinline__ float program_op(int op, float a, float b, float c0, float c1) {
  switch (op) {
#define HMX_OP_CASE(OP, EXPR) \
  case OP:                    \
    return (EXPR);
    HMX_PROGRAM_OPS(HMX_OP_CASE)
#undef HMX_OP_CASE
    default: return a;
  }
}

// N f32 values of one program register.
template <int N>
using program_vec = float __attribute__((ext_vector_type(N)));

// One instruction on n values: the opcode (uniform across the wave) is
// dispatched once for all of them.
template <int N>
__device__ __forceinline__ program_vec<N> program_op_n(int op, program_vec<N> x, program_vec<N> y, float c0,
                                                       float c1) {
  program_vec<N> out;
  switch (op) {
#define HMX_OP_CASE(OP, EXPR)         \
  case OP:                            \
    _Pragma("unroll") for (int i = 0; i < N; ++i) { \
      const float a = x[i], b = y[i]; \
      (void)b;                        \
      out[i] = (EXPR);                \
    }                                 \
    break;
    HMX_PROGRAM_OPS(HMX_OP_CASE)
#undef HMX_OP_CASE
    default: out = x;
  }
  return out;
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

// Runs the program on n values in place (register 0 of value i is v[i],
// register 1 extra[i]): the instructions in turn, each read, computed and
// written for all n values at once, so opcodes and register numbers are
// dispatched once per instruction, not once per value. The register file is
// held as arrays of 8 registers x at most 4 values indexed by the (uniform)
// register number: the compiler keeps arrays of that size in VGPRs and reads
// and writes register k with indexed moves (s_set_gpr_idx), with no branch
// per register (8 x 8 values in one array would go to scratch memory).
template <int N>
__device__ __forceinline__ void run_program_n(const hmx_program& p, float (&v)[N], const float (&extra)[N]) {
  constexpr int H = N > 4 ? 4 : N;  // values per array
  static_assert(N == H || N == 2 * H, "at most two arrays of four values");
  constexpr int R = HMX_PROGRAM_REGS * H;
  float r0[R], r1[N > H ? R : 1];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    r0[i] = v[i];
    r0[H + i] = extra[i];
    if constexpr (N > H) {
      r1[i] = v[H + i];
      r1[H + i] = extra[H + i];
    }
  }
#pragma unroll
  for (int i = 2 * H; i < R; ++i) {
    r0[i] = 0.f;
    if constexpr (N > H) r1[i] = 0.f;
  }
  const int count = __builtin_amdgcn_readfirstlane(p.count);
  // Each instruction is fetched one step ahead, so that its (scalar) load
  // is not waited for at the top of every step.
  hmx_instr next = p.code[0];
#pragma unroll 1
  for (int k = 0; k < count; ++k) {
    const hmx_instr ins = next;
    next = p.code[k + 1 < HMX_PROGRAM_MAX ? k + 1 : k];
    const int a = __builtin_amdgcn_readfirstlane(ins.a) * H, b = __builtin_amdgcn_readfirstlane(ins.b) * H;
    const int d = __builtin_amdgcn_readfirstlane(ins.dst) * H;
    program_vec<N> x, y;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      x[i] = r0[a + i];
      y[i] = r0[b + i];
      if constexpr (N > H) {
        x[H + i] = r1[a + i];
        y[H + i] = r1[b + i];
      }
    }
    const program_vec<N> out = program_op_n<N>(__builtin_amdgcn_readfirstlane(ins.op), x, y, ins.c0, ins.c1);
#pragma unroll
    for (int i = 0; i < H; ++i) {
      r0[d + i] = out[i];
      if constexpr (N > H) r1[d + i] = out[H + i];
    }
  }
  const int res = __builtin_amdgcn_readfirstlane(p.result) * H;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    v[i] = r0[res + i];
    if constexpr (N > H) v[H + i] = r1[res + i];
  }
}

// run_program_n for kernels whose VGPRs are mostly taken (the GEMM
// epilogues): the same instructions in turn, each for all n values at once,
// with the registers in eight separate vector variables read and written in
// the arms of a branch on the (uniform) register number. (One array indexed
// in those arms would be merged by the compiler into a single access at a
// computed index, which puts the register file in scratch memory.)
template <int N>
__device__ __forceinline__ void run_program_branches_n(const hmx_program& p, float (&v)[N], const float (&extra)[N]) {
  using V = program_vec<N>;
  V r0, r1, r2 = V(0.f), r3 = V(0.f), r4 = V(0.f), r5 = V(0.f), r6 = V(0.f), r7 = V(0.f);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    r0[i] = v[i];
    r1[i] = extra[i];
  }
#define HMX_REG_READ(OUT, K)   \
  switch (K) {                 \
    case 0: OUT = r0; break;   \
    case 1: OUT = r1; break;   \
    case 2: OUT = r2; break;   \
    case 3: OUT = r3; break;   \
    case 4: OUT = r4; break;   \
    case 5: OUT = r5; break;   \
    case 6: OUT = r6; break;   \
    case 7: OUT = r7; break;   \
    default: OUT = V(0.f);     \
  }
  const int count = __builtin_amdgcn_readfirstlane(p.count);
  // Each instruction is fetched one step ahead, so that its (scalar) load
  // is not waited for at the top of every step.
  hmx_instr next = p.code[0];
#pragma unroll 1
  for (int k = 0; k < count; ++k) {
    const hmx_instr ins = next;
    next = p.code[k + 1 < HMX_PROGRAM_MAX ? k + 1 : k];
    V a, b;
    HMX_REG_READ(a, __builtin_amdgcn_readfirstlane(ins.a))
    HMX_REG_READ(b, __builtin_amdgcn_readfirstlane(ins.b))
    const V y = program_op_n<N>(__builtin_amdgcn_readfirstlane(ins.op), a, b, ins.c0, ins.c1);
    switch (__builtin_amdgcn_readfirstlane(ins.dst)) {
      case 0: r0 = y; break;
      case 1: r1 = y; break;
      case 2: r2 = y; break;
      case 3: r3 = y; break;
      case 4: r4 = y; break;
      case 5: r5 = y; break;
      case 6: r6 = y; break;
      case 7: r7 = y; break;
      default: break;
    }
  }
  V out;
  HMX_REG_READ(out, __builtin_amdgcn_readfirstlane(p.result))
#undef HMX_REG_READ
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = out[i];
}
static_assert(HMX_PROGRAM_REGS == 8, "the register file's variables");

}  // namespace hmx
