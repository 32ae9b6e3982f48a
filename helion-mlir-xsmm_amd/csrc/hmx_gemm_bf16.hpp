// Register-staged bf16 GEMM kernel template for gfx950 (v_mfma_f32_32x32x16_bf16):
// every bf16 case the direct-to-LDS kernel does not take -- ragged tiles,
// transposed A, the packed B layouts, 128 x 128 tiles.
//
// A workgroup of 4 waves (2 x 2) owns a BM x BN output tile; each wave owns a
// (BM/2) x (BN/2) block of 32 x 32 MFMA fragments. Both operand tiles live in
// LDS K-contiguous (`[rows][BK + 8]` bf16, the 8-element pad makes the
// 16-byte fragment reads conflict-free), double-buffered: the next K tiles'
// global loads are issued into registers ahead of the MFMAs of the current
// one and written to the other LDS buffer after them, so one barrier per K
// tile suffices. Operands that are not K-contiguous in HBM (row-major B,
// transposed A, panel layouts) are transposed in registers on the way (8 x 8
// bf16 blocks through v_perm_b32); VNNI-pair layouts regroup their K pairs
// with no data movement at all.
#pragma once

#include "hmx_gemm_common.hpp"

namespace hmx {
namespace {

// ---------------------------------------------------------------------------
// bf16 operand tile loader: global (layout L) -> registers -> LDS [BR][BK+8].
template <int BR, int BK, int NT, int L, bool GUARD>
struct Bf16Loader {
  static constexpr int KIND = vec_kind<L>();
  static constexpr int PITCH = BK + 8;
  // KIND 0: one 16-byte vector (8 K) per item; KIND 1: an 8-row x 8-K block;
  // KIND 2: a 4-row x 8-K block.
  static constexpr int ITEMS = KIND == 0 ? BR * BK / 8 : KIND == 1 ? BR * BK / 64 : BR * BK / 32;
  static constexpr int PER_THREAD = (ITEMS + NT - 1) / NT;
  static constexpr int REGS = KIND == 0 ? 1 : KIND == 1 ? 8 : 4;
  static_assert(ITEMS % NT == 0 || ITEMS < NT, "tile not divisible among threads");
  uint4 r[PER_THREAD][REGS];

  // Scalar fallback: 8 consecutive elements starting at (row, k) stepping
  // along `dr`/`dk`, zero outside [0, rows) x [0, k_end).
  __device__ __forceinline__ static uint4 gather8(const Operand& o, int64_t row, int64_t k,
                                                  int dr, int dk, int64_t k_end) {
    const uint16_t* p = (const uint16_t*)o.p;
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t rr = row + e * dr, kk = k + e * dk;
      h[e] = (rr < o.rows && kk < k_end) ? p[offset_of<L>(o, rr, kk)] : 0u;
    }
    return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                      h[6] | (h[7] << 16));
  }

  // Whole tiles (no guard): buffer loads, whose offsets split into one
  // per-thread VGPR and a uniform SGPR part for row-major layouts.
  __device__ __forceinline__ void load_whole(__amdgpu_buffer_rsrc_t rsrc, const Operand& o,
                                             int64_t r0, int64_t k0, int tid) {
    constexpr int KV = BK / 8;  // 16-byte vectors per K tile row
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      if (ITEMS < NT && item >= ITEMS) break;
      if constexpr (L == L_KCONTIG) {
        const int32_t voff = (int32_t)(((item / KV) - i * (NT / KV)) * o.ld + (item % KV) * 8) * 2;
        const int32_t soff = (int32_t)(((r0 + i * (NT / KV)) * o.ld + k0) * 2);
        r[i][0] = buffer_load16(rsrc, voff, soff);
      } else if constexpr (L == L_RCONTIG) {
        const int kb = item % KV;
        const int rb = item / KV;
        const int32_t voff = (int32_t)((kb * 8) * o.ld + (rb - i * (NT / KV)) * 8) * 2;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int32_t soff = (int32_t)(((k0 + kk) * o.ld + r0 + i * (NT / KV) * 8) * 2);
          r[i][kk] = buffer_load16(rsrc, voff, soff);
        }
      } else if constexpr (KIND == 1) {
        const int64_t k = k0 + (item % KV) * 8;
        const int64_t row = r0 + (item / KV) * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
          r[i][kk] = buffer_load16(rsrc, (int32_t)(offset_of<L>(o, row, k + kk) * 2), 0);
      } else {
        const int64_t k = k0 + (item % KV) * 8;
        const int64_t row = r0 + (item / KV) * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          r[i][q] = buffer_load16(rsrc, (int32_t)(offset_of<L>(o, row, k + 2 * q) * 2), 0);
      }
    }
  }

  __device__ __forceinline__ void load(const Operand& o, int64_t r0, int64_t k0, int64_t k_end,
                                       int tid) {
    const uint16_t* p = (const uint16_t*)o.p;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      if (ITEMS < NT && item >= ITEMS) break;
      if constexpr (KIND == 0) {
        const int64_t row = r0 + item / (BK / 8);
        const int64_t k = k0 + (item % (BK / 8)) * 8;
        if (!GUARD || (o.vec && row < o.rows && k + 8 <= k_end))
          r[i][0] = *(const uint4*)(p + offset_of<L>(o, row, k));
        else
          r[i][0] = gather8(o, row, k, 0, 1, k_end);
      } else if constexpr (KIND == 1) {
        const int64_t k = k0 + (item % (BK / 8)) * 8;
        const int64_t row = r0 + (item / (BK / 8)) * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          if (!GUARD || (o.vec && row + 8 <= o.rows && k + kk < k_end))
            r[i][kk] = *(const uint4*)(p + offset_of<L>(o, row, k + kk));
          else
            r[i][kk] = gather8(o, row, k + kk, 1, 0, k_end);
        }
      } else {
        const int64_t k = k0 + (item % (BK / 8)) * 8;
        const int64_t row = r0 + (item / (BK / 8)) * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (!GUARD || (o.vec && row + 4 <= o.rows && k + 2 * q + 2 <= k_end)) {
            r[i][q] = *(const uint4*)(p + offset_of<L>(o, row, k + 2 * q));
          } else {
            uint32_t w[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const int64_t rr = row + d, kk = k + 2 * q;
              const uint32_t lo = (rr < o.rows && kk < k_end) ? p[offset_of<L>(o, rr, kk)] : 0u;
              const uint32_t hi =
                  (rr < o.rows && kk + 1 < k_end) ? p[offset_of<L>(o, rr, kk + 1)] : 0u;
              w[d] = lo | (hi << 16);
            }
            r[i][q] = make_uint4(w[0], w[1], w[2], w[3]);
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      if (ITEMS < NT && item >= ITEMS) break;
      const int kcol = (item % (BK / 8)) * 8;
      if constexpr (KIND == 0) {
        const int row = item / (BK / 8);
        *(uint4*)(lds + row * PITCH + kcol) = r[i][0];
      } else if constexpr (KIND == 1) {
        const int row = (item / (BK / 8)) * 8;
        // 8 x 8 transpose: output row j holds K pairs (2d, 2d+1) of column j.
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint4 o;
          if (j & 1) {
            o.x = hi_pair(dw(r[i][0], j >> 1), dw(r[i][1], j >> 1));
            o.y = hi_pair(dw(r[i][2], j >> 1), dw(r[i][3], j >> 1));
            o.z = hi_pair(dw(r[i][4], j >> 1), dw(r[i][5], j >> 1));
            o.w = hi_pair(dw(r[i][6], j >> 1), dw(r[i][7], j >> 1));
          } else {
            o.x = lo_pair(dw(r[i][0], j >> 1), dw(r[i][1], j >> 1));
            o.y = lo_pair(dw(r[i][2], j >> 1), dw(r[i][3], j >> 1));
            o.z = lo_pair(dw(r[i][4], j >> 1), dw(r[i][5], j >> 1));
            o.w = lo_pair(dw(r[i][6], j >> 1), dw(r[i][7], j >> 1));
          }
          *(uint4*)(lds + (row + j) * PITCH + kcol) = o;
        }
      } else {
        const int row = (item / (BK / 8)) * 4;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint4 o = make_uint4(dw(r[i][0], d), dw(r[i][1], d), dw(r[i][2], d), dw(r[i][3], d));
          *(uint4*)(lds + (row + d) * PITCH + kcol) = o;
        }
      }
    }
  }
};

#ifndef HMX_GEMM_SCHED
#define HMX_GEMM_SCHED 1
#endif

// Instruction-class masks of __builtin_amdgcn_sched_group_barrier.
enum : int { SG_VALU = 0x002, SG_MFMA = 0x008, SG_VMEM_READ = 0x020, SG_DS_READ = 0x100, SG_DS_WRITE = 0x200 };

// The order one K step's instructions issue in: the first fragment reads,
// then every MFMA paired with one other instruction -- the next K slice's
// fragment reads, the next-next tile's buffer loads, and the register
// transposes and LDS writes of the next tile -- so that the matrix core
// never waits on an LDS or memory instruction issued just before it.
template <int FM, int FN, int BK, int LOADS, int WRITES, int PERMS>
__device__ __forceinline__ void schedule_k_step() {
#if HMX_GEMM_SCHED
  constexpr int KS = BK / 16, MF = FM * FN, RD = FM + FN;
  constexpr int TOTAL = KS * MF;
  __builtin_amdgcn_sched_group_barrier(SG_DS_READ, RD, 0);
  int loads = LOADS, writes = WRITES, perms = PERMS;
#pragma unroll
  for (int i = 0; i < TOTAL; ++i) {
    const int ks = i / MF, m = i % MF;
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    if (ks + 1 < KS && m < RD) {
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
    } else if (HMX_GEMM_SCHED > 1 && loads > 0 && i < TOTAL / 2) {
      __builtin_amdgcn_sched_group_barrier(SG_VMEM_READ, 1, 0);
      --loads;
    } else if (i >= TOTAL / 2) {
      if (perms > 0) {
        __builtin_amdgcn_sched_group_barrier(SG_VALU, 2, 0);
        perms -= 2;
      }
      if (writes > 0) {
        __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, 1, 0);
        --writes;
      }
    }
  }
#endif
}

template <int BM_, int BN_, int BK_>
struct Bf16Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  static constexpr int NT = 256;           // 4 waves, 2 x 2
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int FM = WM / 32, FN = WN / 32;
  static constexpr int PITCH = BK + 8;
  static constexpr int LDS_ELEMS = 2 * (BM + BN) * PITCH;
};

template <class Cfg, int LA, int LB, bool GUARD>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm_bf16_kernel(GemmArgs g) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NT = Cfg::NT, PITCH = Cfg::PITCH;
  constexpr int FM = Cfg::FM, FN = Cfg::FN;
  __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::LDS_ELEMS];
  // Stage s holds A at lds + s * STAGE and B right after it.
  constexpr int STAGE = (BM + BN) * PITCH;

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, g.xcds, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);

  Operand a = g.a, b = g.b;
  a.p = (const uint16_t*)a.p + batch * g.stride_a;
  b.p = (const uint16_t*)b.p + batch * g.stride_b;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Two register staging sets: tile t + 2's global loads are issued while
  // tile t is multiplied, so each load has two K steps to arrive.
  Bf16Loader<BM, BK, NT, LA, GUARD> la0, la1;
  Bf16Loader<BN, BK, NT, LB, GUARD> lb0, lb1;

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int ktiles = (int)((k_end - k_begin + BK - 1) / BK);
  // K offset of tile t, clamped to the last tile: the loads past the end
  // re-read it, in bounds, so the loop needs no conditional loads.
  auto k_of = [&](int t) { return k_begin + (int64_t)min(t, ktiles - 1) * BK; };
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.p, a.bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(b.p, b.bytes);
  auto fetch = [&](auto& ld_a, auto& ld_b, int t) {
    if constexpr (GUARD) {
      ld_a.load(a, m0, k_of(t), k_end, tid);
      ld_b.load(b, n0, k_of(t), k_end, tid);
    } else {
      ld_a.load_whole(ra, a, m0, k_of(t), tid);
      ld_b.load_whole(rb, b, n0, k_of(t), tid);
    }
  };
  if (ktiles > 0) {
    fetch(la0, lb0, 0);
    fetch(la1, lb1, 1);
    la0.store(lds, tid);
    lb0.store(lds + BM * PITCH, tid);
  }
  __syncthreads();

  // Fragment read offsets: row lane % 32 of the fragment, K half lane / 32.
  const int frag_row = lane & 31, frag_k = (lane >> 5) * 8;
  auto multiply = [&](const uint16_t* stage) {
    const uint16_t* As = stage + (wm * Cfg::WM + frag_row) * PITCH + frag_k;
    const uint16_t* Bs = stage + BM * PITCH + (wn * Cfg::WN + frag_row) * PITCH + frag_k;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *(const bf16x8_t*)(As + i * 32 * PITCH + ks * 16);
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[j] = *(const bf16x8_t*)(Bs + j * 32 * PITCH + ks * 16);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  };
  uint16_t* const stage0 = lds;
  uint16_t* const stage1 = lds + STAGE;
  using LoadA = Bf16Loader<BM, BK, NT, LA, GUARD>;
  using LoadB = Bf16Loader<BN, BK, NT, LB, GUARD>;
  constexpr int kLoads = LoadA::PER_THREAD * LoadA::REGS + LoadB::PER_THREAD * LoadB::REGS;
  constexpr int kWrites = LoadA::PER_THREAD * (LoadA::KIND == 0 ? 1 : LoadA::KIND == 1 ? 8 : 4) +
                          LoadB::PER_THREAD * (LoadB::KIND == 0 ? 1 : LoadB::KIND == 1 ? 8 : 4);
  constexpr int kPerms = (LoadA::KIND == 1 ? LoadA::PER_THREAD * 32 : 0) +
                         (LoadB::KIND == 1 ? LoadB::PER_THREAD * 32 : 0);
  int kt = 0;
  for (; kt + 2 <= ktiles; kt += 2) {
    // Even step: tile kt from stage 0; tile kt + 1 (set 1) goes to stage 1.
    __builtin_amdgcn_sched_barrier(0);
    fetch(la0, lb0, kt + 2);
    __builtin_amdgcn_sched_barrier(0);
    multiply(stage0);
#if !HMX_GEMM_SCHED
    __builtin_amdgcn_sched_barrier(0);
#endif
    la1.store(stage1, tid);
    lb1.store(stage1 + BM * PITCH, tid);
    schedule_k_step<FM, FN, BK, kLoads, kWrites, kPerms>();
    __syncthreads();
    // Odd step: tile kt + 1 from stage 1; tile kt + 2 (set 0) goes to stage 0.
    __builtin_amdgcn_sched_barrier(0);
    fetch(la1, lb1, kt + 3);
    __builtin_amdgcn_sched_barrier(0);
    multiply(stage1);
#if !HMX_GEMM_SCHED
    __builtin_amdgcn_sched_barrier(0);
#endif
    la0.store(stage0, tid);
    lb0.store(stage0 + BM * PITCH, tid);
    schedule_k_step<FM, FN, BK, kLoads, kWrites, kPerms>();
    __syncthreads();
  }
  // An odd tile count leaves the last tile in stage 0.
  if (kt < ktiles) {
    multiply(stage0);
    __syncthreads();
  }

  static_assert(4 * 32 * epi_pitch<Cfg::WN>() * 4 <= Cfg::LDS_ELEMS * 2, "epilogue does not fit LDS");
  epilogue<FM, FN, Cfg::WM, Cfg::WN, GUARD>(g, (float*)lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
}

template <class Cfg, int LA, int LB>
void launch_bf16(const GemmArgs& g, bool guard, dim3 grid, hipStream_t s) {
  if (guard)
    launch(gemm_bf16_kernel<Cfg, LA, LB, true>, grid, Cfg::NT, s, g);
  else
    launch(gemm_bf16_kernel<Cfg, LA, LB, false>, grid, Cfg::NT, s, g);
}

// Row-major or transposed A and B (L_KCONTIG / L_RCONTIG).
template <class Cfg>
void dispatch_bf16_plain(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s) {
  if (la == L_KCONTIG) {
    if (lb == L_KCONTIG)
      launch_bf16<Cfg, L_KCONTIG, L_KCONTIG>(g, guard, grid, s);
    else
      launch_bf16<Cfg, L_KCONTIG, L_RCONTIG>(g, guard, grid, s);
  } else {
    if (lb == L_KCONTIG)
      launch_bf16<Cfg, L_RCONTIG, L_KCONTIG>(g, guard, grid, s);
    else
      launch_bf16<Cfg, L_RCONTIG, L_RCONTIG>(g, guard, grid, s);
  }
}

}  // namespace

// Per-unit launchers (hmx_gemm_bf16_256.hip, hmx_gemm_bf16_128.hip,
// hmx_gemm_bf16_packed.hip), split so the instantiations compile in parallel.
void launch_gemm_bf16_256(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s);
void launch_gemm_bf16_128(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s);
void launch_gemm_bf16_packed(const GemmArgs& g, int lb, bool guard, dim3 grid, hipStream_t s);

}  // namespace hmx
