// Direct-to-LDS building blocks of the gfx950 GEMM kernels
// (hmx_gemm_dma.hip): buffer resources, the
// `buffer_load_dwordx4 ... lds` copy of 16 bytes per lane into LDS, its wait,
// the LDS tile swizzles and the transposing LDS read.
//
// These loads and their waits are inline assembly: the compiler would
// otherwise wait for every outstanding LDS load (vmcnt(0)) before any LDS
// read, which leaves nothing in flight. Loads complete in issue order, so the
// compiler's own waits for other memory operations stay correct.
#pragma once

#include "hmx_gemm_common.hpp"

namespace hmx {
namespace {

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4_t make_srd(const void* p, int32_t bytes) {
  const uint64_t a = (uint64_t)p;
  return i32x4_t{(int32_t)(uint32_t)a, (int32_t)((a >> 32) & 0xffff), bytes, 0x00020000};
}

// One 16-byte-per-lane load from buffer `srd` at voff + soff bytes into LDS
// bytes [lds, lds + 1024) (lane l at lds + 16 l). An LDS load must not read M0
// in the cycle after the SALU write of it (one wait state, the s_nop). The
// kernel has no other use of M0, so clobbering it is safe. NT: the load is
// non-temporal (streamed past the caches' retention), for operand data no
// other workgroup reads: the split-K bf16 bmm of config 5 runs 203 -> 189 us
// with it, while GEMMs whose tiles share panels through L2 run 15 % slower.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(i32x4_t srd, int32_t voff, int32_t soff, uint32_t lds) {
  // The scalar offset and the LDS address are uniform by construction; saying
  // so keeps them in SGPRs where the compiler cannot prove it (run-time
  // compilation of the VNNI-panel loads), and costs nothing where it can.
  soff = __builtin_amdgcn_readfirstlane(soff);
  lds = __builtin_amdgcn_readfirstlane(lds);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
                 :: "v"(voff), "s"(srd), "s"(soff), "s"(lds) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :: "v"(voff), "s"(srd), "s"(soff), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ int swz_k(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz_n(int r) { return ((r & 3) << 1) ^ ((r & 3) << 2); }
__device__ __forceinline__ int swz64(int r) { return (r >> 1) & 7; }
// Row-major B tiles of the 16x16x32 kernel: swz_n, with bit 3 of the K row
// also flipping chunk bit 1. One transposing fragment read covers rows
// r .. r + 3 and r + 8 .. r + 11 in its two 16-lane halves; with swz_n alone
// both halves met the same banks (a two-way conflict on every read).
__device__ __forceinline__ int bswz(int r) { return swz_n(r) ^ ((r >> 2) & 2); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ bf16x4_t lds_read_tr(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)p);
}

}  // namespace
}  // namespace hmx
