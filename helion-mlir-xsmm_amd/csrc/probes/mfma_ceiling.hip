// MFMA throughput ceiling of one MI355X by operand data: every wave runs the
// GEMM kernels' per-wave block (4 A x 4 B fragments of
// v_mfma_f32_32x32x16_bf16, 16 accumulators, one wave per SIMD on 256 CUs)
// with no memory traffic. Constant operands toggle few multiplier bits;
// random bf16 operands (the benchmarks' U[-1,1] data) draw more power, and the
// clock the power limit allows sets the dense-bf16 ceiling a GEMM can reach.
//
//   hipcc --offload-arch=gfx950 -O3 -o mfma_ceiling mfma_ceiling.hip && ./mfma_ceiling
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// mode 0: constant 1 + {0, .25, .5, .75}; mode 1: U[-1, 1].
__device__ __bf16 operand(uint32_t h, int mode) {
  if (mode == 0) return (__bf16)(1.0f + (h & 3) * 0.25f);
  return (__bf16)(((h >> 8) * (1.0f / 16777216.0f)) * 2.f - 1.f);
}

template <int MODE>
__global__ __launch_bounds__(256, 1) void mfma_block(float* out, int iters) {
  bf16x8_t a[4], b[4];
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  for (int i = 0; i < 4; ++i)
    for (int e = 0; e < 8; ++e) {
      a[i][e] = operand(mix(t * 64 + i * 8 + e), MODE);
      b[i][e] = operand(mix(0x9e3779b9u ^ (t * 64 + i * 8 + e)), MODE);
    }
  f32x16_t acc[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 16; ++e) s += acc[i][j][e];
  out[t] = s;
}

// The same block on the f32 MFMA (v_mfma_f32_32x32x2_f32, one value per lane
// per operand), the instruction of the f32 GEMM.
template <int MODE>
__global__ __launch_bounds__(256, 1) void mfma_block_f32(float* out, int iters) {
  float a[4], b[4];
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  for (int i = 0; i < 4; ++i) {
    a[i] = (float)operand(mix(t * 8 + i), MODE);
    b[i] = (float)operand(mix(0x9e3779b9u ^ (t * 8 + i)), MODE);
    if (MODE == 1) {  // full 24-bit mantissas, not bf16 values
      a[i] += (mix(t * 8 + i + 4) >> 8) * (1.0f / 4294967296.0f);
      b[i] -= (mix(0x85ebca6bu ^ (t * 8 + i)) >> 8) * (1.0f / 4294967296.0f);
    }
  }
  f32x16_t acc[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j)
      for (int e = 0; e < 16; ++e) s += acc[i][j][e];
  out[t] = s;
}

template <typename K>
static int run(const char* name, K kernel, int iters, double flops_per_mfma = 32768.0) {
  float* out = nullptr;
  if (hipMalloc(&out, 256 * 256 * sizeof(float)) != hipSuccess) return 1;
  hipEvent_t s, e;
  hipEventCreate(&s);
  hipEventCreate(&e);
  kernel<<<256, 256>>>(out, iters);
  if (hipDeviceSynchronize() != hipSuccess) return 1;
  for (int rep = 0; rep < 3; ++rep) {
    hipEventRecord(s);
    kernel<<<256, 256>>>(out, iters);
    hipEventRecord(e);
    hipEventSynchronize(e);
    float ms = 0.f;
    hipEventElapsedTime(&ms, s, e);
    const double flops = 1024.0 * iters * 16 * flops_per_mfma;
    printf("%-28s %9.3f ms %8.1f TFLOP/s\n", name, ms, flops / ms / 1e9);
  }
  fflush(stdout);
  hipFree(out);
  return 0;
}

int main() {
  int rc = 0;
  rc |= run("constant operands", mfma_block<0>, 50000);
  rc |= run("random U[-1,1] operands", mfma_block<1>, 50000);
  rc |= run("random, 1.5 ms runs", mfma_block<1>, 5000);
  rc |= run("f32 constant operands", mfma_block_f32<0>, 10000, 4096.0);
  rc |= run("f32 random operands", mfma_block_f32<1>, 10000, 4096.0);
  return rc;
}
