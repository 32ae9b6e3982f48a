// HBM read ceiling of the GEMM kernels' operand stream on one MI355X: 256
// workgroups of 8 waves (one per CU) stream 4 MiB each into LDS with the
// kernels' direct-to-LDS loads (`buffer_load_dwordx4 ... lds`, 1 KiB per load),
// in stages of SB bytes with D stages in flight (D + 1 LDS buffers), and do
// nothing else. Two address patterns:
//   contig: each stage is SB contiguous bytes;
//   bmm:    the split-K bmm of [16, 256, 65536] @ [16, 65536, 256] bf16, one
//           workgroup per (slice, K chunk of 4096): each stage is SB / 512
//           bytes of each of the 256 A rows (128 KiB apart) and SB / 1024
//           contiguous 512-byte rows of B.
//
//   hipcc --offload-arch=gfx950 -O3 -o stream_ceiling stream_ceiling.hip && ./stream_ceiling
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                            \
  do {                                                                      \
    hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                 \
      std::printf("%s: %s\n", #x, hipGetErrorString(e_));                  \
      std::exit(1);                                                         \
    }                                                                       \
  } while (0)

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

constexpr int64_t kRowBytes = 65536 * 2;                        // A row stride
constexpr int64_t kBBase = 16LL * 256 * kRowBytes;              // B after A: 512 MiB
constexpr int64_t kTotal = kBBase + 16LL * 65536 * 256 * 2;     // 1 GiB
constexpr int64_t kPerBlock = 4LL << 20;                        // bytes each workgroup reads

__device__ __forceinline__ i32x4_t make_srd(const void* p, int32_t bytes) {
  const uint64_t a = (uint64_t)p;
  return i32x4_t{(int32_t)(uint32_t)a, (int32_t)((a >> 32) & 0xffff), bytes, 0x00020000};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(i32x4_t srd, int32_t voff, int32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(srd), "s"(soff), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

template <bool BMM, int SB, int D>
__global__ __launch_bounds__(512, 1) void stream(const uint8_t* src, float* sink) {
  constexpr int NB = D + 1, LPW = SB / 8 / 1024;  // LDS buffers; 1 KiB loads per wave per stage
  constexpr int stages = (int)(kPerBlock / SB);
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NB * SB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, blk = blockIdx.x;
  const i32x4_t srd = make_srd(src, (int32_t)kTotal);
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + w * (SB / 8);
  auto issue = [&](int t) {
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      int32_t voff, soff;
      if constexpr (!BMM) {
        voff = lane * 16;
        soff = (int32_t)(blk * kPerBlock + (int64_t)t * SB + w * (SB / 8) + q * 1024);
      } else {
        const int slice = blk / 16, chunk = blk % 16;
        constexpr int AB = SB / 512;    // bytes of each A row per stage
        constexpr int RPL = 1024 / AB;  // A rows per load
        constexpr int LA = LPW / 2;     // A loads per wave (32 rows)
        if (q < LA) {
          voff = (int32_t)((lane / (AB / 16)) * kRowBytes + (lane % (AB / 16)) * 16);
          soff = (int32_t)(slice * 256 * kRowBytes + chunk * 4096 * 2 + (w * 32 + q * RPL) * kRowBytes +
                           (int64_t)t * AB);
        } else {
          const int qb = q - LA;
          voff = (lane >> 5) * 512 + (lane & 31) * 16;
          soff = (int32_t)(kBBase + slice * 65536LL * 512 + chunk * 4096LL * 512 +
                           ((int64_t)t * (SB / 1024) + w * (SB / 8192) + qb * 2) * 512);
        }
      }
      lds_dma16(srd, voff, __builtin_amdgcn_readfirstlane(soff),
                __builtin_amdgcn_readfirstlane(base + (t % NB) * SB + q * 1024));
    }
  };
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < D; ++t) issue(t);
  for (int t = 0; t < stages; ++t) {
    if (t + D < stages) {
      issue(t + D);  // into the buffer read in step t - 1 (before its second barrier)
      asm volatile("s_waitcnt vmcnt(%0)" :: "n"(D * LPW) : "memory");  // stage t landed
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    acc += *(const float*)(lds + (t % NB) * SB + threadIdx.x * (SB / 512));
    __syncthreads();
  }
  if (acc == 12345.f) sink[blk] = acc;  // keeps the LDS reads
}

template <bool BMM, int SB, int D>
void run(const uint8_t* src, float* sink) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  for (int i = 0; i < 3; ++i) stream<BMM, SB, D><<<256, 512>>>(src, sink);
  CHECK(hipDeviceSynchronize());
  const int reps = 10;
  CHECK(hipEventRecord(a));
  for (int i = 0; i < reps; ++i) stream<BMM, SB, D><<<256, 512>>>(src, sink);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  ms /= reps;
  const double bytes = 256.0 * kPerBlock;
  std::printf("%-7s stage %2d KiB, %d in flight  %7.1f us  %5.2f TB/s\n", BMM ? "bmm" : "contig", SB / 1024, D,
              ms * 1e3, bytes / (ms * 1e-3) / 1e12);
  std::fflush(stdout);
}

int main() {
  uint8_t* src = nullptr;
  float* sink = nullptr;
  CHECK(hipMalloc(&src, kTotal));
  CHECK(hipMalloc(&sink, 256 * sizeof(float)));
  CHECK(hipMemset(src, 1, kTotal));
  run<false, 65536, 1>(src, sink);
  run<false, 32768, 1>(src, sink);
  run<false, 32768, 3>(src, sink);
  run<false, 16384, 3>(src, sink);
  run<false, 16384, 8>(src, sink);
  run<true, 65536, 1>(src, sink);
  run<true, 32768, 1>(src, sink);
  run<true, 32768, 3>(src, sink);
  CHECK(hipFree(src));
  CHECK(hipFree(sink));
  return 0;
}
