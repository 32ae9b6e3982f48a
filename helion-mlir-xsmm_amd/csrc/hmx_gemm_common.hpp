// Shared pieces of the GEMM translation units (hmx_gemm_bf16_*.hip,
// hmx_gemm_dma.hip, hmx_gemm_f32.hip and the host side hmx_gemm.cpp): operand
// layouts, the kernel argument block, the workgroup -> tile mapping, the fused
// epilogues, and the launchers each kernel unit exports.
#pragma once

#include <type_traits>

#include "hmx_device.hpp"

namespace hmx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Operand layouts (A: rows are M, B: rows are N; both indexed (row, k)).
enum : int {
  L_KCONTIG = 0,      // row * ld + k
  L_RCONTIG = 1,      // k * ld + row
  L_VNNI_PANELS = 2,  // [R/P, Kp/2, P, 2]
  L_BLOCKED_VNNI = 3, // [R/32, Kp/32, 16, 32, 2]
  L_PANELS = 4,       // [R/P, Kp, P]
  L_BLOCKED = 5,      // [R/32, Kp/32, 32, 32]
};

// How a layout's 16-byte vectors run: along K, along rows, or 4 rows x 2 K.
template <int L>
constexpr int vec_kind() {
  return L == L_KCONTIG ? 0 : (L == L_VNNI_PANELS || L == L_BLOCKED_VNNI) ? 2 : 1;
}

struct Operand {
  const void* p;   // this batch slice
  int64_t ld;      // line stride (row-major layouts)
  int64_t rows;    // logical extent along rows (M or N)
  int64_t panel;   // panel width (panel layouts)
  int64_t kpad;    // padded K (packed layouts)
  bool vec;        // 16-byte loads allowed (alignment of base and lines)
  int32_t bytes;   // extent of one batch slice in bytes (buffer loads; < 2^31)
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// A buffer resource over one operand slice: loads past `bytes` return zeros
// instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, int32_t voff, int32_t soff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int L>
__device__ __forceinline__ int64_t offset_of(const Operand& o, int64_t r, int64_t k) {
  if constexpr (L == L_KCONTIG) return r * o.ld + k;
  if constexpr (L == L_RCONTIG) return k * o.ld + r;
  if constexpr (L == L_VNNI_PANELS)
    return (((r / o.panel) * (o.kpad >> 1) + (k >> 1)) * o.panel + (r % o.panel)) * 2 + (k & 1);
  if constexpr (L == L_BLOCKED_VNNI)
    return ((((r >> 5) * (o.kpad >> 5) + (k >> 5)) * 16 + ((k & 31) >> 1)) * 32 + (r & 31)) * 2 +
           (k & 1);
  if constexpr (L == L_PANELS) return ((r / o.panel) * o.kpad + k) * o.panel + (r % o.panel);
  if constexpr (L == L_BLOCKED)
    return (((r >> 5) * (o.kpad >> 5) + (k >> 5)) * 32 + (k & 31)) * 32 + (r & 31);
  return 0;
}

__device__ __forceinline__ uint32_t lo_pair(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);  // {x.lo16, y.lo16}
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);  // {x.hi16, y.hi16}
}
__device__ __forceinline__ uint32_t dw(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// ---------------------------------------------------------------------------
struct GemmArgs {
  Operand a, b;
  int64_t stride_a, stride_b;  // batch strides (elements)
  void* c;
  int64_t ldc, stride_c, stride_split;
  int c_dtype;
  int64_t m, n, k, k_chunk;
  const void* bias;
  const void* scale;
  const void* shift;
  int vec_dtype;
  int act;
  float act_arg;
  int tiles_m, tiles_n;
  // Nonzero: each workgroup walks its K chunk from a stage of its own
  // (wrapping), for split-K grids whose workgroups share no operand data.
  int k_stagger;
  // The device's compute units and XCDs (workgroups are dealt to the XCDs
  // in turn; each XCD has its own L2).
  int cus, xcds;
  // act == HMX_EPI_PROGRAM: the epilogue program (last: the kernels that do
  // not run programs never read it).
  hmx_program prog;
};

// blockIdx.x -> (tile_m, tile_n). Consecutive workgroups are dealt to the
// device's XCDs in turn; renumbering them so that each XCD gets one
// contiguous range, then walking that range in groups of kGroupM tile rows,
// makes the tiles that share A rows and B columns run on the same XCD and its
// L2.
// `bid` is the workgroup's index in the launch's run of this tile grid (a run
// starting at a multiple of xcds, so that bid % xcds is still its XCD).
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int xcds, int& tm, int& tn) {
  constexpr int kGroupM = 4;
  const int nb = tiles_m * tiles_n;
  if (xcds > 1 && nb % xcds == 0) bid = (bid % xcds) * (nb / xcds) + bid / xcds;
  const int per_group = kGroupM * tiles_n;
  const int group = bid / per_group;
  const int first_m = group * kGroupM;
  const int gm = min(kGroupM, tiles_m - first_m);
  const int in_group = bid % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int xcds, int& tm, int& tn) {
  tile_coords((int)blockIdx.x, tiles_m, tiles_n, xcds, tm, tn);
}

__device__ __forceinline__ void column_vectors(const GemmArgs& g, int64_t col, bool in,
                                               float& bias, float& scale, float& shift) {
  bias = (g.bias && in) ? load_any(g.bias, g.vec_dtype, col) : 0.f;
  scale = (g.scale && in) ? load_any(g.scale, g.vec_dtype, col) : 1.f;
  shift = (g.shift && in) ? load_any(g.shift, g.vec_dtype, col) : 0.f;
}

// Bias, scale and shift of columns col .. col + 3 (columns from n on:
// identity values): one 8-byte (bf16) or 16-byte (f32) load per vector where
// all four columns are below n and the load is aligned, else element by
// element.
__device__ __forceinline__ void column_vectors4(const GemmArgs& g, int64_t col, int64_t n, float (&cb)[4],
                                                float (&cs)[4], float (&ch)[4]) {
  const bool bf = g.vec_dtype == HMX_DTYPE_BF16;
  auto four = [&](const void* p, float id, float (&out)[4]) {
    if (!p) {
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] = id;
      return;
    }
    const uint16_t* h = (const uint16_t*)p + col;
    const float* f = (const float*)p + col;
    if (col + 4 <= n && (bf ? ((uintptr_t)h & 7) : ((uintptr_t)f & 15)) == 0) {
      if (bf) {
        const uint2 v = *(const uint2*)h;
        out[0] = bf16_bits_to_f32((uint16_t)(v.x & 0xffff));
        out[1] = bf16_bits_to_f32((uint16_t)(v.x >> 16));
        out[2] = bf16_bits_to_f32((uint16_t)(v.y & 0xffff));
        out[3] = bf16_bits_to_f32((uint16_t)(v.y >> 16));
      } else {
        const float4 v = *(const float4*)f;
        out[0] = v.x;
        out[1] = v.y;
        out[2] = v.z;
        out[3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] = col + e < n ? load_any(p, g.vec_dtype, col + e) : id;
    }
  };
  four(g.bias, 0.f, cb);
  four(g.scale, 1.f, cs);
  four(g.shift, 0.f, ch);
}


// f(std::integral_constant<int, I>) for the runtime index i == I (0 <= i <
// N). A loop the compiler leaves rolled (one around an epilogue program's
// interpreter is too large to unroll) reads the accumulators through it, by a
// constant index in each branch: indexed by the loop counter they would be
// moved to scratch memory.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void with_index(int i, F&& f) {
  if constexpr (I + 1 < N) {
    if (i == I)
      f(std::integral_constant<int, I>{});
    else
      with_index<N, I + 1>(i, f);
  } else {
    f(std::integral_constant<int, I>{});
  }
}

// The epilogue's activation on N values in place: a named code, or with
// PROG (kernels instantiated for epilogue programs only, so the others do not
// carry the interpreter's registers) the program.
template <int N, bool PROG>
__device__ __forceinline__ void activate_all(const GemmArgs& g, float (&v)[N]) {
  if (PROG && g.act == HMX_EPI_PROGRAM) {
    // The branch-per-register interpreter: the indexed register file of the
    // row kernels spills in the 256-VGPR GEMM kernels (config 4 with a
    // 4-instruction program: 1000 -> 1405 us).
    const float none[N] = {};
    run_program_branches_n<N>(g.prog, v, none);
  } else {
    // One switch per value: dispatching once for all N values unrolls every
    // activation N times, and the registers that takes spilled (GELU-tanh
    // linear 830 -> 940 us).
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = apply_activation(g.act, v[i], g.act_arg);
  }
}

// Epilogue, staged through LDS (free once the K loop is done). Each wave owns
// a region of 32 x (WN + 8) f32; for each of its FM fragment rows it writes
// the accumulators there (element e of lane l of a 32 x 32 fragment is row
// 8*(e/4) + 4*(l/32) + e%4, column l % 32), then reads them back four
// columns per lane to apply bias, scale, shift and the activation and store
// C with 8- or 16-byte coalesced writes.
template <int WN>
constexpr int epi_pitch() { return WN + 8; }

// Activation classes compiled into the register epilogue. ACT_ANY: any
// other named activation, ACT_PROG: an epilogue program, both finished by the
// LDS-staged epilogue (separate instantiations: only ACT_PROG carries the
// interpreter's registers). ACT_JIT: the epilogue compiled in at run time
// (hmx_jit.cpp) as hmx_jit_epilogue, finished in registers like ReLU.
enum : int { ACT_ID = 0, ACT_RELU = 1, ACT_SILU = 2, ACT_ANY = 3, ACT_PROG = 4, ACT_JIT = 5 };

// The staged class for an epilogue code that is not identity, ReLU or SiLU.
constexpr bool staged_act(int act) { return act == ACT_ANY || act == ACT_PROG; }

// The run-time compiled epilogue of ACT_JIT kernels: f(value, extra). Only
// the sources that hmx_jit.cpp compiles define it; the library's own
// kernels never instantiate ACT_JIT.
__device__ float hmx_jit_epilogue(float x, float extra);

template <int ACT>
__device__ __forceinline__ float activate(float v) {
  if constexpr (ACT == ACT_RELU) return apply_activation(HMX_EPI_RELU, v, 0.f);
  if constexpr (ACT == ACT_SILU) return apply_activation(HMX_EPI_SILU, v, 0.f);
  if constexpr (ACT == ACT_JIT) return hmx_jit_epilogue(v, 0.f);
  return v;
}

// Exchange with the neighbouring lane (lane ^ 1) through DPP, no LDS.
__device__ __forceinline__ float swap_pair(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1 /* quad_perm [1,0,3,2] */, 0xF, 0xF, false));
}

#ifndef HMX_EPI_STREAM
#define HMX_EPI_STREAM 1
#endif

// A 4-byte store of C. C is written once and not read back by the kernel:
// the non-temporal hint keeps the writes from allocating cache lines.
__device__ __forceinline__ void store_c32(void* p, uint32_t v) {
#if HMX_EPI_STREAM
  __builtin_nontemporal_store(v, (uint32_t*)p);
#else
  *(uint32_t*)p = v;
#endif
}

// Register epilogue: each lane finishes its own accumulators (column
// lane % 32 of each fragment: bias, scale, shift, activation) and stores them
// directly. bf16 pairs: rows r and r + 1 of adjacent columns are exchanged
// between lanes 2c and 2c + 1, so every lane writes one 4-byte word (two
// columns of one row); f32 lanes write their own 4-byte values.
template <int FM, int FN, int WM, int WN, bool GUARD, int ACT, bool BF16>
__device__ __forceinline__ void epilogue_direct(const GemmArgs& g, int split, int batch, int64_t m0,
                                                int64_t n0, int wm, int wn, int lane, bool pair_ok,
                                                const f32x16_t (&acc)[FM][FN]) {
  const int64_t off = split * g.stride_split + batch * g.stride_c;
  const bool odd = lane & 1;
  (void)pair_ok;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * WN + j * 32 + (lane & 31);
    const bool col_in = !GUARD || col < g.n;
    float bias, scale, shift;
    column_vectors(g, col, col_in, bias, scale, shift);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int64_t row0 = m0 + wm * WM + i * 32 + 4 * (lane >> 5);
      if constexpr (BF16) {
        uint16_t* c = (uint16_t*)g.c + off;
        if constexpr (!GUARD) {
          // Whole tile: 4-byte stores of column pairs.
          const int64_t pcol = col & ~(int64_t)1;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int e0 = 2 * q, e1 = 2 * q + 1;
            const float v0 = activate<ACT>((acc[i][j][e0] + bias) * scale + shift);
            const float v1 = activate<ACT>((acc[i][j][e1] + bias) * scale + shift);
            const float recv = swap_pair(odd ? v0 : v1);
            const int64_t row = row0 + 8 * (e0 >> 2) + (e0 & 3) + (odd ? 1 : 0);
            store_c32(c + row * g.ldc + pcol, odd ? pack_bf16x2(recv, v1) : pack_bf16x2(v0, recv));
          }
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int64_t row = row0 + 8 * (e >> 2) + (e & 3);
            const float v = activate<ACT>((acc[i][j][e] + bias) * scale + shift);
            if (col_in && row < g.m) c[row * g.ldc + col] = (uint16_t)f32_to_bf16_bits(v);
          }
        }
      } else {
        float* c = (float*)g.c + off;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t row = row0 + 8 * (e >> 2) + (e & 3);
          const float v = activate<ACT>((acc[i][j][e] + bias) * scale + shift);
          if (!GUARD || (col_in && row < g.m)) store_c32(c + row * g.ldc + col, __float_as_uint(v));
        }
      }
    }
  }
}

template <int FM, int FN, int WM, int WN, bool GUARD, bool PROG = false>
__device__ __forceinline__ void epilogue_staged(const GemmArgs& g, float* lds, int split, int batch,
                                         int64_t m0, int64_t n0, int wm, int wn, int wave,
                                         int lane, const f32x16_t (&acc)[FM][FN]) {
  constexpr int P = epi_pitch<WN>();
  float* ep = lds + wave * 32 * P;
  const int64_t off = split * g.stride_split + batch * g.stride_c;
  const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
  const bool vec_ok = (g.ldc % 4 == 0) &&
                      ((((uintptr_t)g.c) & (bf16 ? 7 : 15)) == 0) && (off % 4 == 0);
  const int64_t col0 = n0 + wn * WN;
  // A lane's 4 columns are the same in every step below (64 is a multiple of
  // WN / 4): their bias, scale and shift are loaded once (inside the loop the
  // stores to C keep the compiler from hoisting the loads).
  static_assert(64 % (WN / 4) == 0, "a lane's columns are the same in every step");
  const int cq = (lane % (WN / 4)) * 4;
  float cb[4], cs[4], ch[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) column_vectors(g, col0 + cq + t, !GUARD || col0 + cq + t < g.n, cb[t], cs[t], ch[t]);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    with_index<FM>(i, [&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          ep[(8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * P + j * 32 + (lane & 31)] = acc[I][j][e];
    });
    __syncthreads();
    const int64_t row0 = m0 + wm * WM + i * 32;
    for (int idx = lane; idx < 32 * (WN / 4); idx += 64) {
      const int r = idx / (WN / 4);
      const int64_t row = row0 + r, col = col0 + cq;
      if (GUARD && row >= g.m) continue;
      const float4 q = *(const float4*)(ep + r * P + cq);
      float v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = (v[t] + cb[t]) * cs[t] + ch[t];
      activate_all<4, PROG>(g, v);
      const int64_t o = off + row * g.ldc + col;
      if ((!GUARD || col + 4 <= g.n) && vec_ok) {
        if (bf16)
          *(uint2*)((uint16_t*)g.c + o) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        else
          *(float4*)((float*)g.c + o) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (GUARD && col + t >= g.n) break;
          if (bf16)
            ((uint16_t*)g.c)[o + t] = (uint16_t)f32_to_bf16_bits(v[t]);
          else
            ((float*)g.c)[o + t] = v[t];
        }
      }
    }
    __syncthreads();
  }
}

// Epilogue dispatch: identity, ReLU and SiLU store from registers; other
// activations go through the LDS-staged path.
template <int FM, int FN, int WM, int WN, bool GUARD>
__device__ __forceinline__ void epilogue(const GemmArgs& g, float* lds, int split, int batch,
                                         int64_t m0, int64_t n0, int wm, int wn, int wave,
                                         int lane, const f32x16_t (&acc)[FM][FN]) {
  const bool bf16 = g.c_dtype == HMX_DTYPE_BF16;
  const int64_t off = split * g.stride_split + batch * g.stride_c;
  const bool pair_ok = (g.ldc % 2 == 0) && (off % 2 == 0) && ((((uintptr_t)g.c) & 3) == 0);
#define HMX_DIRECT(ACT)                                                                          \
  do {                                                                                           \
    if (bf16)                                                                                    \
      epilogue_direct<FM, FN, WM, WN, GUARD, ACT, true>(g, split, batch, m0, n0, wm, wn, lane,   \
                                                         pair_ok, acc);                          \
    else                                                                                         \
      epilogue_direct<FM, FN, WM, WN, GUARD, ACT, false>(g, split, batch, m0, n0, wm, wn, lane,  \
                                                          pair_ok, acc);                         \
  } while (0)
  if (!GUARD && !pair_ok && bf16) {
    epilogue_staged<FM, FN, WM, WN, GUARD>(g, lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
    return;
  }
  switch (g.act) {
    case HMX_EPI_IDENTITY: HMX_DIRECT(ACT_ID); break;
    case HMX_EPI_RELU: HMX_DIRECT(ACT_RELU); break;
    case HMX_EPI_SILU: HMX_DIRECT(ACT_SILU); break;
    default:
      epilogue_staged<FM, FN, WM, WN, GUARD>(g, lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
  }
#undef HMX_DIRECT
}

#ifndef __HIPCC_RTC__
// Kernel launchers, one translation unit each. `la` / `lb` are L_* layouts
// of A and B; `guard` selects the kernels that check every edge.
// hmx_gemm_bf16_*.hip: register-staged bf16 kernel, tiles 256 x 256 or 128 x 128
// (packed B layouts at 256 x 256 only).
void launch_gemm_bf16(const GemmArgs& g, int tile_bm, int la, int lb, bool guard, dim3 grid,
                      hipStream_t s);
// hmx_gemm_dma.hip: direct-to-LDS bf16 kernels (64-wide K stages when K
// chunks are whole 64-element stages, else 32-wide); whole 256 x 256 tiles, A
// K-contiguous, B K-contiguous, row-major or (64-wide only) packed, identity /
// ReLU / SiLU epilogue.
void launch_gemm_bf16_dma(const GemmArgs& g, int lb, dim3 grid, hipStream_t s);
// The 64-wide direct-to-LDS kernel on 256 x 128 tiles (four waves, B
// [N, K] or [K, N]): the columns past the last whole round of 256 x 256 tiles.
void launch_gemm_bf16_dma_narrow(const GemmArgs& g, int lb, dim3 grid, hipStream_t s);
// Both in one launch where the 16x16x32 kernel runs both with a named
// activation: workgroups 0 .. head_blocks - 1 take head's 256 x 256 tiles,
// the rest rest's 256 x 128 tiles, so the tail's workgroups start as the last
// round's free their CUs, with no kernel boundary between. False (nothing
// launched) where it does not apply.
bool launch_gemm_bf16_dma_rounds(const GemmArgs& head, const GemmArgs& rest, int lb, unsigned head_blocks,
                                 unsigned rest_blocks, hipStream_t s);
// The 64-wide direct-to-LDS kernel with A stored [K, M] (trans_a): whole
// 256 x 256 tiles, K chunks of whole 64-element stages, B K-contiguous or
// row-major.
void launch_gemm_bf16_dma_ta(const GemmArgs& g, int lb, dim3 grid, hipStream_t s);
// The 64-wide direct-to-LDS kernel on 128 x 128 tiles (four waves of 64 x 64,
// B [N, K] or [K, N], K chunks of whole 64-element stages), whole or ragged.
void launch_gemm_bf16_dma128(const GemmArgs& g, int lb, dim3 grid, hipStream_t s);
// Skinny products: M <= 64, row-major A, B [N, K], batch 1, K a multiple of
// 64, operand spans below 2^31 bytes, 16-byte aligned rows; one workgroup per
// 32 columns of C, K split over its waves, any epilogue, C bf16 or f32.
void launch_gemm_bf16_skinny(const GemmArgs& g, hipStream_t s);
// Whether the 64-wide direct-to-LDS kernel reads this packed B in place
// (VNNI panels, blocked VNNI, K-major panels, 32 x 32 blocks).
bool gemm_bf16_dma_packed_ok(const GemmArgs& g, int lb);
// hmx_gemm_f32.hip: f32 kernel, tiles 64 x 64, 128 x 128 or (split-K
// partials only) 256 x 256; and the fixed-order split-K reduction into C.
// hmx_gemm_dma.hip: direct-to-LDS f32 kernel; whole 256 x 256 tiles of
// split-K partials (identity epilogue, f32 C), A K-contiguous, B K-contiguous
// or row-major, K chunks of whole 32-element stages.
void launch_gemm_f32_dma(const GemmArgs& g, int lb, dim3 grid, hipStream_t s);
void launch_gemm_f32(const GemmArgs& g, int tile_bm, int la, int lb, bool guard, dim3 grid,
                     hipStream_t s);
void launch_splitk_reduce(const float* partials, int splits, int64_t batch, const GemmArgs& r,
                          bool vec4, hipStream_t s);
// hmx_jit.cpp: the 16x16x32 kernel (layout lb, bf16 or f32 C, ragged or
// whole tiles of bm x bn, nw waves, `stages` K stages) with g's epilogue --
// a program or a named activation -- compiled into its register epilogue at
// run time. HMX_OK, or HMX_ERR_UNSUPPORTED when run-time compilation is off
// (HMX_JIT=0) or failed: the caller then launches the interpreter.
int launch_mi16_jit(const GemmArgs& g, int lb, bool bf16, bool ragged, int bm, int bn, int nw, int stages,
                    dim3 grid, hipStream_t s);
// hmx_jit.cpp: launch_gemm_bf16_dma_rounds's one launch of whole rounds of
// 256 x 256 tiles (head) and the 256 x 128 tail (rest) with g's epilogue
// compiled in at run time; HMX_OK or HMX_ERR_UNSUPPORTED as launch_mi16_jit.
int launch_mi16_rounds_jit(const GemmArgs& head, const GemmArgs& rest, int lb, bool bf16, unsigned head_blocks,
                           unsigned rest_blocks, hipStream_t stream);
// While a JitCompileOff lives on a thread, that thread's launches use kernels
// already compiled but compile and load none (hipRTC and module loading
// allocate): a kernel not yet compiled is HMX_ERR_UNSUPPORTED, the prebuilt
// path runs, and a later call may still compile it. For hmx_gemm_noalloc.
struct JitCompileOff {
  explicit JitCompileOff(bool on);
  ~JitCompileOff();
  JitCompileOff(const JitCompileOff&) = delete;
  JitCompileOff& operator=(const JitCompileOff&) = delete;
  bool was;
  bool on;
};
#endif  // __HIPCC_RTC__

}  // namespace hmx
