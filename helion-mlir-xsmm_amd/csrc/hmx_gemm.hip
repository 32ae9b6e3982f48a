// GEMM kernels for gfx950: bf16 x bf16 -> f32 on v_mfma_f32_32x32x16_bf16 and
// f32 x f32 -> f32 on v_mfma_f32_32x32x2_f32, with the epilogue
// act(((A @ B) + bias) * scale + shift) fused before the single rounding to C,
// batch slices on grid z and deterministic split-K on grid y.
//
// bf16 kernel. A workgroup of 4 waves (2 x 2) owns a BM x BN output tile;
// each wave owns a (BM/2) x (BN/2) block of 32 x 32 MFMA fragments. Both
// operand tiles live in LDS K-contiguous (`[rows][BK + 8]` bf16, the 8-element
// pad makes the 16-byte fragment reads conflict-free), double-buffered: the
// next K tile's global loads are issued into registers before the MFMAs of
// the current one and written to the other LDS buffer after them, so one
// barrier per K tile suffices. Operands that are not K-contiguous in HBM
// (row-major B, transposed A, panel layouts) are transposed in registers on
// the way (8 x 8 bf16 blocks through v_perm_b32); VNNI-pair layouts regroup
// their K pairs with no data movement at all.
//
// f32 kernel. Same structure with BK = 32 and the f32 MFMA, whose operands
// are one value per lane: LDS keeps each operand in its HBM orientation and
// fragments are gathered with 4-byte (or 16-byte, when K-contiguous) reads.
#include <type_traits>

#include "hmx_device.hpp"

namespace hmx {
namespace {

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
};

// blockIdx.x -> (tile_m, tile_n). Consecutive workgroups are dealt to the 8
// XCDs in turn; renumbering them so that each XCD gets one contiguous range,
// then walking that range in groups of kGroupM tile rows, makes the tiles
// that share A rows and B columns run on the same XCD and its L2.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int kXcds = 8, kGroupM = 4;
  const int nb = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if (nb % kXcds == 0) bid = (bid % kXcds) * (nb / kXcds) + bid / kXcds;
  const int per_group = kGroupM * tiles_n;
  const int group = bid / per_group;
  const int first_m = group * kGroupM;
  const int gm = min(kGroupM, tiles_m - first_m);
  const int in_group = bid % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

__device__ __forceinline__ void column_vectors(const GemmArgs& g, int64_t col, bool in,
                                               float& bias, float& scale, float& shift) {
  bias = (g.bias && in) ? load_any(g.bias, g.vec_dtype, col) : 0.f;
  scale = (g.scale && in) ? load_any(g.scale, g.vec_dtype, col) : 1.f;
  shift = (g.shift && in) ? load_any(g.shift, g.vec_dtype, col) : 0.f;
}


// Epilogue, staged through LDS (free once the K loop is done). Each wave owns
// a region of 32 x (WN + 8) f32; for each of its FM fragment rows it writes
// the accumulators there (element e of lane l of a 32 x 32 fragment is row
// 8*(e/4) + 4*(l/32) + e%4, column l % 32), then reads them back four
// columns per lane to apply bias, scale, shift and the activation and store
// C with 8- or 16-byte coalesced writes.
template <int WN>
constexpr int epi_pitch() { return WN + 8; }

// Activation classes compiled into the register epilogue.
enum : int { ACT_ID = 0, ACT_RELU = 1, ACT_SILU = 2 };

template <int ACT>
__device__ __forceinline__ float activate(float v) {
  if constexpr (ACT == ACT_RELU) return apply_activation(HMX_EPI_RELU, v, 0.f);
  if constexpr (ACT == ACT_SILU) return apply_activation(HMX_EPI_SILU, v, 0.f);
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

template <int FM, int FN, int WM, int WN, bool GUARD>
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
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        ep[(8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * P + j * 32 + (lane & 31)] = acc[i][j][e];
    __syncthreads();
    const int64_t row0 = m0 + wm * WM + i * 32;
    for (int idx = lane; idx < 32 * (WN / 4); idx += 64) {
      const int r = idx / (WN / 4), cq = (idx % (WN / 4)) * 4;
      const int64_t row = row0 + r, col = col0 + cq;
      if (GUARD && row >= g.m) continue;
      const float4 q = *(const float4*)(ep + r * P + cq);
      float v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bool in = !GUARD || col + t < g.n;
        float bias, scale, shift;
        column_vectors(g, col + t, in, bias, scale, shift);
        v[t] = apply_activation(g.act, (v[t] + bias) * scale + shift, g.act_arg);
      }
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
  tile_coords(g.tiles_m, g.tiles_n, tm, tn);
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

// ---------------------------------------------------------------------------
// bf16 kernel for whole 256 x 256 tiles of row-major A and a B that is
// either K-contiguous ([N, K]) or row-major ([K, N]): operand tiles go from
// memory straight into LDS (`buffer_load_dwordx4 ... lds`), with no VGPR
// staging and no LDS write instructions. Four LDS stages of BK = 32 keep
// three tiles in flight.
//
// LDS tiles are unpadded: one such load fills 1 KiB of LDS contiguously
// (lane l at byte 16 l), so bank conflicts are avoided by XOR-swizzling
// 16-byte chunks instead -- the lane that fills slot c of tile row r fetches
// global chunk c ^ swz(r).
//  * A, and K-contiguous B: [256 rows][32 k], 64-byte rows (4 chunks),
//    swz_k(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1). A fragment read (16 bytes:
//    row lane % 32, chunk 2 ks + lane / 32) then meets distinct banks whether
//    LDS serves 8 or 16 lanes per cycle.
//  * row-major B: [32 k][256 n], 512-byte rows (32 chunks),
//    swz_n(r) = ((r & 3) << 1) ^ ((r & 3) << 2). Fragments come from
//    ds_read_b64_tr_b16, which transposes within each group of 16 lanes:
//    lane j receives, as its element e, element j % 4 of the 8 bytes lane
//    4 e + j / 4 addressed. Lane s of a group addresses row k0 + s / 4 at
//    columns n0 + 4 (s % 4) .. + 3, so lane j ends with B[k0 .. k0 + 3][n0 + j],
//    the MFMA's K-ordered operand; two such reads make the 8-value operand.
//    The 4 rows x 2 (16 lanes) or 4 (32 lanes) chunks touched per pass land
//    on distinct banks.
//
// These loads and their waits are inline assembly: the compiler would
// otherwise wait for every outstanding LDS load (vmcnt(0)) before any LDS
// read, which leaves nothing in flight. Loads complete in issue order, so the
// compiler's own waits for other memory operations stay correct.
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4_t make_srd(const void* p, int32_t bytes) {
  const uint64_t a = (uint64_t)p;
  return i32x4_t{(int32_t)(uint32_t)a, (int32_t)((a >> 32) & 0xffff), bytes, 0x00020000};
}

// One 16-byte-per-lane load from buffer `srd` at voff + soff bytes into LDS
// bytes [lds, lds + 1024) (lane l at lds + 16 l). An LDS load must not read M0
// in the cycle after the SALU write of it (one wait state, the s_nop). The
// kernel has no other use of M0, so clobbering it is safe.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(i32x4_t srd, int32_t voff, int32_t soff, uint32_t lds) {
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

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ bf16x4_t lds_read_tr(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)p);
}

// One instantiation per B orientation, register-epilogue class and C dtype:
// a single straight-line epilogue keeps the accumulators out of scratch.
template <int LB, int ACT, bool BF16>
__global__ __launch_bounds__(256, 1) void gemm_bf16_dma_kernel(GemmArgs g) {
  constexpr bool BT = LB == L_RCONTIG;             // B row-major [K, N]
  constexpr int BM = 256, BN = 256, BK = 32, S = 4;
  constexpr int ROWB = BK * 2;                     // bytes per K-contiguous tile row
  constexpr int NROWB = BN * 2;                    // bytes per row-major B tile row
  constexpr int A_BYTES = BM * ROWB;               // 16 KiB
  constexpr int STAGE = A_BYTES + BN * BK * 2;     // 32 KiB
  constexpr int FM = 4, FN = 4, WM = 128, WN = 128;
  constexpr int LOADS = 8;                         // DMA instructions per wave per tile
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE];

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);
  const int ktiles = (int)((k_end - k_begin) / BK);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const i32x4_t srd_a = make_srd((const uint16_t*)g.a.p + batch * g.stride_a, g.a.bytes);
  const i32x4_t srd_b = make_srd((const uint16_t*)g.b.p + batch * g.stride_b, g.b.bytes);
  // Wave w loads 16-row blocks 4w .. 4w + 3 of the A tile: lane l fills slot
  // l % 4 of block row l / 4. Byte offsets below 2^31: the operands' byte
  // ranges are.
  const int drow = lane >> 2;
  const int32_t voff_a = (int32_t)((drow * g.a.ld + ((lane & 3) ^ swz_k(drow)) * 8) * 2);
  const int32_t soff_a = (int32_t)((m0 + wave * 64) * g.a.ld * 2);
  const int32_t blk_a = (int32_t)(16 * g.a.ld * 2);
  // B: K-contiguous as A; row-major in pairs of rows 8w + 2q, 8w + 2q + 1
  // (q < 4), lane l filling slot l % 32 of row l / 32 of the pair.
  int32_t voff_b0, voff_b1, soff_b, blk_b;
  if constexpr (BT) {
    const int r = lane >> 5, c = lane & 31;
    voff_b0 = (int32_t)((r * g.b.ld + (c ^ swz_n(r)) * 8) * 2);      // even q
    voff_b1 = (int32_t)((r * g.b.ld + (c ^ swz_n(r + 2)) * 8) * 2);  // odd q
    soff_b = (int32_t)((wave * 8 * g.b.ld + n0) * 2);
    blk_b = (int32_t)(2 * g.b.ld * 2);
  } else {
    voff_b0 = voff_b1 = (int32_t)((drow * g.b.ld + ((lane & 3) ^ swz_k(drow)) * 8) * 2);
    soff_b = (int32_t)((n0 + wave * 64) * g.b.ld * 2);
    blk_b = (int32_t)(16 * g.b.ld * 2);
  }
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + wave * 4 * 1024;

  // DMA q (< 8) of tile t: A blocks for q < 4, then B.
  auto dma = [&](int t, int q) {
    const int64_t k0 = k_begin + (int64_t)min(t, ktiles - 1) * BK;
    const uint32_t st = lds_w + (uint32_t)((t % S) * STAGE);
    if (q < 4) {
      lds_dma16(srd_a, voff_a, soff_a + q * blk_a + (int32_t)(k0 * 2), st + q * 1024);
    } else {
      const int32_t kb = BT ? (int32_t)(k0 * g.b.ld * 2) : (int32_t)(k0 * 2);
      lds_dma16(srd_b, (q & 1) ? voff_b1 : voff_b0, soff_b + (q - 4) * blk_b + kb,
                st + A_BYTES + (q - 4) * 1024);
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment reads. A (and K-contiguous B): row lane % 32 of the fragment,
  // chunk 2 ks + lane / 32.
  const int frow = lane & 31, fk = lane >> 5, fswz = swz_k(frow);
  const uint8_t* a_frag = lds + (wm * WM + frow) * ROWB;
  const uint8_t* b_frag = lds + A_BYTES + (wn * WN + frow) * ROWB;
  // Row-major B: lane s of 16-lane group gi addresses row 8 (gi / 2) + s / 4
  // (+ 16 ks, + 4 for the second read) and the chunk holding columns
  // wn * 128 + 32 j + 16 (gi % 2) + 4 (s % 4).
  int b_tr[FN];
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int v = (2 * (gi & 1) + ((sl & 3) >> 1)) ^ swz_n(sl >> 2);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      b_tr[j] = A_BYTES + (8 * (gi >> 1) + (sl >> 2)) * NROWB + (wn * 16 + ((4 * j) ^ v)) * 16 + 8 * (sl & 1);
  }
  auto a_read = [&](int stage, int ks, int i) -> bf16x8_t {
    return *(const bf16x8_t*)(a_frag + stage * STAGE + i * 32 * ROWB + ((2 * ks + fk) ^ fswz) * 16);
  };
  auto b_read = [&](int stage, int ks, int j) -> bf16x8_t {
    if constexpr (BT) {
      const uint8_t* p = lds + stage * STAGE + b_tr[j] + 16 * ks * NROWB;
      return __builtin_shufflevector(lds_read_tr(p), lds_read_tr(p + 4 * NROWB), 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      return *(const bf16x8_t*)(b_frag + stage * STAGE + j * 32 * ROWB + ((2 * ks + fk) ^ fswz) * 16);
    }
  };

  // The host launches this kernel only with at least one K tile per split.
  bf16x8_t a0[FM], b0[FN], a1[FM], b1[FN];
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int q = 0; q < LOADS; ++q) dma(t, q);
  wait_vmem<2 * LOADS>();  // tile 0 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) a0[i] = a_read(0, 0, i);
#pragma unroll
  for (int j = 0; j < FN; ++j) b0[j] = b_read(0, 0, j);

  for (int t = 0; t < ktiles; ++t) {
    // Tiles t + 1 and t + 2 are in flight: wait for t + 1, then the barrier
    // publishes it and frees stage (t + 3) % S (last read in step t - 1).
    // The barrier carries no LDS fence: every LDS read of the freed stage
    // was consumed by an MFMA of step t - 1 before it.
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(LOADS) : "memory");
    const int cur = t % S, nxt = t + 1 < ktiles ? (t + 1) % S : cur;
    // 32 MFMA slots per step, each paired with at most one other memory
    // operation: slots 0-7 read k-step 1's fragments, slots 8-15 issue the
    // DMA of tile t + 3, slots 16-23 read the next tile's k-step 0 fragments
    // (a quarter step ahead of the barrier that follows).
#pragma unroll
    for (int x = 0; x < 32; ++x) {
      __builtin_amdgcn_sched_barrier(0);
      const int f = x & 7;
      if (x < 8) {
        if (f < 4) a1[f] = a_read(cur, 1, f);
        else b1[f - 4] = b_read(cur, 1, f - 4);
      } else if (x < 16) {
        dma(t + 3, f);
      } else if (x < 24) {
        if (f < 4) a0[f] = a_read(nxt, 0, f);
        else b0[f - 4] = b_read(nxt, 0, f - 4);
      }
      const int idx = x & 15, i = idx >> 2, j = idx & 3;
      if (x < 16)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[i], b0[j], acc[i][j], 0, 0, 0);
      else
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[i], b1[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_vmem<0>();  // no load into LDS outlives the loop
  epilogue_direct<FM, FN, WM, WN, false, ACT, BF16>(g, split, batch, m0, n0, wm, wn, lane, true, acc);
}

// ---------------------------------------------------------------------------
// f32 kernel.
template <int BM_, int BN_, int BK_>
struct F32Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  // 256 x 256 tiles run 8 waves (2 per SIMD, 2 x 4 over the tile) so that one
  // wave's LDS traffic and barrier hide behind the other's MFMAs.
  static constexpr int NT = BM == 256 ? 512 : 256;
  static constexpr int WAVES_N = NT / 128;
  static constexpr int WM = BM / 2, WN = BN / WAVES_N;
  static constexpr int FM = WM / 32, FN = WN / 32;
};

// LDS image of an f32 operand tile in its HBM orientation: K-contiguous
// `[BR][BK + 4]` or row-contiguous `[BK][BR + 8]` (pads against bank
// conflicts of the fragment reads).
template <int BR, int BK, int NT, int L, bool GUARD>
struct F32Loader {
  static constexpr bool KC = L == L_KCONTIG;
  static constexpr int PITCH = KC ? BK + 4 : BR + 8;
  static constexpr int ELEMS = KC ? BR * PITCH : BK * PITCH;
  static constexpr int ITEMS = BR * BK / 4;
  static constexpr int PER_THREAD = ITEMS / NT;
  static_assert(ITEMS % NT == 0, "tile not divisible among threads");
  uint4 r[PER_THREAD];

  __device__ __forceinline__ void load(const Operand& o, int64_t r0, int64_t k0, int64_t k_end,
                                       int tid) {
    const float* p = (const float*)o.p;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      int64_t row, k;
      if constexpr (KC) {
        row = r0 + item / (BK / 4);
        k = k0 + (item % (BK / 4)) * 4;
      } else {
        k = k0 + item / (BR / 4);
        row = r0 + (item % (BR / 4)) * 4;
      }
      const bool fits = KC ? (row < o.rows && k + 4 <= k_end) : (row + 4 <= o.rows && k < k_end);
      if (!GUARD || (o.vec && fits)) {
        r[i] = *(const uint4*)(p + offset_of<L>(o, row, k));
      } else {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t rr = KC ? row : row + e, kk = KC ? k + e : k;
          v[e] = (rr < o.rows && kk < k_end) ? p[offset_of<L>(o, rr, kk)] : 0.f;
        }
        r[i] = Elem<float>::pack(v);
      }
    }
  }

  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int item = i * NT + tid;
      if constexpr (KC)
        *(uint4*)(lds + (item / (BK / 4)) * PITCH + (item % (BK / 4)) * 4) = r[i];
      else
        *(uint4*)(lds + (item / (BR / 4)) * PITCH + (item % (BR / 4)) * 4) = r[i];
    }
  }

  // The 4 values lane group g feeds MFMAs s = 0..3 of K step k8: K index
  // k8 + 4g + s, row `row` of the tile.
  __device__ __forceinline__ static void frag(const float* lds, int row, int k, float (&v)[4]) {
    if constexpr (KC) {
      const float4 q = *(const float4*)(lds + row * PITCH + k);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) v[s] = lds[(k + s) * PITCH + row];
    }
  }
};

template <class Cfg, int LAY_A, int LAY_B, bool GUARD>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm_f32_kernel(GemmArgs g) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NT = Cfg::NT;
  constexpr int FM = Cfg::FM, FN = Cfg::FN;
  using LA = F32Loader<BM, BK, NT, LAY_A, GUARD>;
  using LB = F32Loader<BN, BK, NT, LAY_B, GUARD>;
  __shared__ __attribute__((aligned(16))) float lds[2 * (LA::ELEMS + LB::ELEMS)];
  constexpr int STAGE = LA::ELEMS + LB::ELEMS;

  int tm, tn;
  tile_coords(g.tiles_m, g.tiles_n, tm, tn);
  const int split = blockIdx.y, batch = blockIdx.z;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t k_begin = (int64_t)split * g.k_chunk;
  const int64_t k_end = min(g.k, k_begin + g.k_chunk);

  Operand a = g.a, b = g.b;
  a.p = (const float*)a.p + batch * g.stride_a;
  b.p = (const float*)b.p + batch * g.stride_b;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;

  LA la;
  LB lb;
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int ktiles = (int)((k_end - k_begin + BK - 1) / BK);
  if (ktiles > 0) {
    la.load(a, m0, k_begin, k_end, tid);
    lb.load(b, n0, k_begin, k_end, tid);
    la.store(lds, tid);
    lb.store(lds + LA::ELEMS, tid);
  }
  __syncthreads();

  const int frag_row = lane & 31, frag_k = (lane >> 5) * 4;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    // Prefetch the next K tile (the last iteration re-reads its own, in
    // bounds): unconditional, so the staging registers stay registers.
    const int64_t kn = k_begin + (int64_t)min(kt + 1, ktiles - 1) * BK;
    la.load(a, m0, kn, k_end, tid);
    lb.load(b, n0, kn, k_end, tid);
#pragma unroll
    for (int k8 = 0; k8 < BK; k8 += 8) {
      float av[FM][4], bv[FN][4];
#pragma unroll
      for (int i = 0; i < FM; ++i) LA::frag(lds + cur * STAGE, wm * Cfg::WM + i * 32 + frag_row, k8 + frag_k, av[i]);
#pragma unroll
      for (int j = 0; j < FN; ++j) LB::frag(lds + cur * STAGE + LA::ELEMS, wn * Cfg::WN + j * 32 + frag_row, k8 + frag_k, bv[j]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bv[j][s], acc[i][j], 0, 0, 0);
    }
    la.store(lds + (cur ^ 1) * STAGE, tid);
    lb.store(lds + (cur ^ 1) * STAGE + LA::ELEMS, tid);
    __syncthreads();
  }

  if constexpr (BM == 256) {
    // Launched only for split-K partials: identity into f32, no vectors.
    epilogue_direct<FM, FN, Cfg::WM, Cfg::WN, GUARD, ACT_ID, false>(g, split, batch, m0, n0, wm, wn, lane,
                                                                     true, acc);
  } else {
    static_assert(4 * 32 * epi_pitch<Cfg::WN>() <= 2 * STAGE, "epilogue does not fit LDS");
    epilogue<FM, FN, Cfg::WM, Cfg::WN, GUARD>(g, lds, split, batch, m0, n0, wm, wn, wave, lane, acc);
  }
}

// ---------------------------------------------------------------------------
// Split-K reduction: out[b, i, j] = epilogue(sum_s ws[s, b, i, j]) with s in
// increasing order, so the result never depends on scheduling. V consecutive
// columns per thread: 16-byte partial loads and 8/16-byte C stores when rows
// and C keep that alignment (V = 4), else one element (V = 1).
template <int V>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws,
                                                            int splits, int64_t batch,
                                                            GemmArgs g) {
  const int64_t mn = g.m * g.n;
  const int64_t total = batch * mn / V;
  const int64_t split_stride = batch * mn;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t idx = t * V;
    float acc[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = 0.f;
    for (int sp = 0; sp < splits; ++sp) {
      const float* p = ws + sp * split_stride + idx;
      if constexpr (V == 4) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        acc[0] += q.x;
        acc[1] += q.y;
        acc[2] += q.z;
        acc[3] += q.w;
      } else {
        acc[0] += p[0];
      }
    }
    const int64_t b = idx / mn, rem = idx % mn;
    const int64_t row = rem / g.n, col = rem % g.n;
    float v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float bias, scale, shift;
      column_vectors(g, col + e, true, bias, scale, shift);
      v[e] = apply_activation(g.act, (acc[e] + bias) * scale + shift, g.act_arg);
    }
    const int64_t off = b * g.stride_c + row * g.ldc + col;
    if (g.c_dtype == HMX_DTYPE_BF16) {
      uint16_t* c = (uint16_t*)g.c + off;
      if constexpr (V == 4)
        __builtin_nontemporal_store(
            (uint64_t)pack_bf16x2(v[0], v[1]) | ((uint64_t)pack_bf16x2(v[2], v[3]) << 32), (uint64_t*)c);
      else
        *c = (uint16_t)f32_to_bf16_bits(v[0]);
    } else {
      float* c = (float*)g.c + off;
      if constexpr (V == 4)
        store16_stream(c, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                     __float_as_uint(v[3])));
      else
        *c = v[0];
    }
  }
}

// ---------------------------------------------------------------------------
// Host side: tile table, planning, dispatch.

struct TileChoice {
  int bm, bn, bk;
};

// Instantiated workgroup tiles, largest first.
constexpr TileChoice kBf16Tiles[] = {{256, 256, 64}, {128, 128, 64}};
constexpr TileChoice kF32Tiles[] = {{128, 128, 32}};
// The f32 tile long-K split-K products of whole 256 x 256 tiles take (see
// make_plan): one workgroup per CU reading each operand once.
constexpr TileChoice kF32Big = {256, 256, 16};
constexpr int kCus = 256;  // MI355X compute units

int layout_code(int b_layout) {
  switch (b_layout) {
    case HMX_B_ROW: return L_RCONTIG;
    case HMX_B_TRANS: return L_KCONTIG;
    case HMX_B_VNNI_PANELS: return L_VNNI_PANELS;
    case HMX_B_BLOCKED_VNNI: return L_BLOCKED_VNNI;
    case HMX_B_PANELS: return L_PANELS;
    case HMX_B_BLOCKED: return L_BLOCKED;
  }
  return -1;
}

struct Plan {
  TileChoice tile;
  int splits;
  int64_t k_chunk;
  int64_t workspace_bytes;
  // Row-major bf16 B is first transposed to [N, K] in the workspace (at
  // offset 0, bt_bytes long) when enough output rows reuse it: the K-contiguous
  // kernel path then reads it without register transposes.
  bool transpose_b;
  int64_t bt_bytes;
};

// Output rows from which a row-major bf16 B is transposed once up front.
constexpr int64_t kTransposeMinRows = 512;

// Split K while the grid holds fewer workgroups than fit the CUs at once
// (one 256 x 256 workgroup per CU, four of the smaller tiles), each chunk
// keeps at least 8 K tiles, and the partials (written and read again as f32)
// stay within a quarter of the operand traffic and the workspace limit.
int auto_splits(TileChoice tile, int64_t tiles, int64_t m, int64_t n, int64_t k, int64_t batch,
                int64_t esz, int64_t max_ws) {
  const int64_t kt = ceil_div(k, tile.bk);
  const int64_t operand_bytes = batch * (m + n) * k * esz;
  const int64_t resident = (tile.bm == 256 ? 1 : 4) * kCus;
  int splits = 1;
  for (;;) {
    const int s2 = splits * 2;
    if (tiles * splits >= resident || kt / s2 < 8) break;
    const int64_t need = (int64_t)s2 * batch * m * n * 4;
    if ((max_ws >= 0 && need > max_ws) || 2 * need > operand_bytes / 4) break;
    splits = s2;
  }
  return splits;
}

int make_plan(int ab_dtype, int64_t m, int64_t n, int64_t k, int64_t batch, int trans_a,
              int b_layout, int splits, int64_t max_ws, int tile_m, int tile_n, int tile_k,
              Plan& plan) {
  const bool bf16 = ab_dtype == HMX_DTYPE_BF16;
  const TileChoice* table = bf16 ? kBf16Tiles : kF32Tiles;
  const int count = bf16 ? (int)(sizeof(kBf16Tiles) / sizeof(TileChoice))
                         : (int)(sizeof(kF32Tiles) / sizeof(TileChoice));
  // Packed B layouts are instantiated for the first tile only.
  const bool packed = b_layout != HMX_B_ROW && b_layout != HMX_B_TRANS;
  int pick = -1;
  if (tile_m > 0 || tile_n > 0 || tile_k > 0) {
    for (int i = 0; i < count && pick < 0; ++i) {
      if ((tile_m <= 0 || table[i].bm <= tile_m) && (tile_n <= 0 || table[i].bn <= tile_n) &&
          (tile_k <= 0 || table[i].bk <= tile_k))
        pick = i;
    }
    if (pick < 0) pick = count - 1;
  } else {
    // The largest tile that still gives every CU a workgroup; else the smallest.
    pick = count - 1;
    for (int i = 0; i < count; ++i) {
      const int64_t tiles = ceil_div(m, table[i].bm) * ceil_div(n, table[i].bn) * batch;
      if (tiles >= kCus) { pick = i; break; }
    }
    // Long-K bf16 products of whole 256 x 256 tiles that split-K can spread
    // over every CU take the big tile: it reads each operand once (half the
    // operand traffic of 128 x 128 tiles), and that traffic bounds them.
    const int64_t big_tiles = (m / 256) * (n / 256) * batch;
    const TileChoice big = bf16 ? table[0] : kF32Big;
    if (!packed && !trans_a && m % 256 == 0 && n % 256 == 0 && k % big.bk == 0 && big_tiles > 0 &&
        big_tiles < kCus &&
        big_tiles * (splits > 0 ? splits
                                : auto_splits(big, big_tiles, m, n, k, batch, bf16 ? 2 : 4, max_ws)) >=
            kCus)
      pick = bf16 ? 0 : -2;
  }
  if (packed && bf16) pick = 0;
  plan.tile = pick == -2 ? kF32Big : table[pick];
  const int64_t tiles = ceil_div(m, plan.tile.bm) * ceil_div(n, plan.tile.bn) * batch;
  const int64_t kt = ceil_div(k, plan.tile.bk);
  if (splits == 0) splits = auto_splits(plan.tile, tiles, m, n, k, batch, bf16 ? 2 : 4, max_ws);
  if (splits < 1) splits = 1;
  if (splits > 1) {
    // Whole K tiles per chunk; no empty chunks.
    plan.k_chunk = ceil_div(kt, splits) * plan.tile.bk;
    splits = (int)ceil_div(k, plan.k_chunk);
  } else {
    plan.k_chunk = k;
  }
  plan.splits = splits;
  const int64_t partial_bytes = splits > 1 ? (int64_t)splits * batch * m * n * 4 : 0;
  plan.bt_bytes = ceil_div(n * k * 2, 256) * 256;
  // Whole 256 x 256 tiles of row-major A read row-major B in place
  // (direct-to-LDS kernel); other bf16 shapes with enough rows read it
  // transposed up front.
  const bool dma_reads_b = plan.tile.bm == 256 && !trans_a && m % 256 == 0 && n % 256 == 0 &&
                           k % plan.tile.bk == 0 && plan.k_chunk % plan.tile.bk == 0;
  plan.transpose_b = bf16 && b_layout == HMX_B_ROW && !dma_reads_b && batch == 1 &&
                     m >= kTransposeMinRows &&
                     n * k * 2 < INT32_MAX &&
                     (max_ws < 0 || plan.bt_bytes + partial_bytes <= max_ws);
  if (!plan.transpose_b) plan.bt_bytes = 0;
  plan.workspace_bytes = plan.bt_bytes + partial_bytes;
  return HMX_OK;
}

template <int V>
using IntC = std::integral_constant<int, V>;

template <class Cfg, int LA, int LB>
void launch_bf16(const GemmArgs& g, bool guard, dim3 grid, hipStream_t s) {
  if (guard)
    gemm_bf16_kernel<Cfg, LA, LB, true><<<grid, Cfg::NT, 0, s>>>(g);
  else
    gemm_bf16_kernel<Cfg, LA, LB, false><<<grid, Cfg::NT, 0, s>>>(g);
}

template <class Cfg>
void dispatch_bf16(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s) {
  if (la == L_KCONTIG) {
    switch (lb) {
      case L_KCONTIG: launch_bf16<Cfg, L_KCONTIG, L_KCONTIG>(g, guard, grid, s); break;
      case L_RCONTIG: launch_bf16<Cfg, L_KCONTIG, L_RCONTIG>(g, guard, grid, s); break;
      default:
        if constexpr (Cfg::BM == kBf16Tiles[0].bm && Cfg::BN == kBf16Tiles[0].bn) {
          switch (lb) {
            case L_VNNI_PANELS: launch_bf16<Cfg, L_KCONTIG, L_VNNI_PANELS>(g, guard, grid, s); break;
            case L_BLOCKED_VNNI: launch_bf16<Cfg, L_KCONTIG, L_BLOCKED_VNNI>(g, guard, grid, s); break;
            case L_PANELS: launch_bf16<Cfg, L_KCONTIG, L_PANELS>(g, guard, grid, s); break;
            case L_BLOCKED: launch_bf16<Cfg, L_KCONTIG, L_BLOCKED>(g, guard, grid, s); break;
          }
        }
    }
  } else {
    if (lb == L_KCONTIG)
      launch_bf16<Cfg, L_RCONTIG, L_KCONTIG>(g, guard, grid, s);
    else
      launch_bf16<Cfg, L_RCONTIG, L_RCONTIG>(g, guard, grid, s);
  }
}

// The direct-to-LDS bf16 kernel serves every case it can unless the
// environment sets HMX_GEMM_DMA=0 (which selects the register-staged kernel,
// for comparison).
bool dma_enabled() {
  static const bool on = [] {
    const char* e = getenv("HMX_GEMM_DMA");
    return !(e && e[0] == '0');
  }();
  return on;
}

// The direct-to-LDS kernel finishes C with the register epilogue only:
// identity, ReLU or SiLU, and 4-byte aligned column pairs for bf16 C.
bool dma_direct_ok(const GemmArgs& g) {
  const bool act_ok = g.act == HMX_EPI_IDENTITY || g.act == HMX_EPI_RELU || g.act == HMX_EPI_SILU;
  const bool pair_ok = g.c_dtype != HMX_DTYPE_BF16 ||
                       (g.ldc % 2 == 0 && g.stride_c % 2 == 0 && g.stride_split % 2 == 0 &&
                        (((uintptr_t)g.c) & 3) == 0);
  return act_ok && pair_ok && g.k_chunk % 32 == 0 && g.k > 0;
}

template <int LB, bool BF16>
void launch_bf16_dma_c(const GemmArgs& g, dim3 grid, hipStream_t s) {
  switch (g.act) {
    case HMX_EPI_RELU: gemm_bf16_dma_kernel<LB, ACT_RELU, BF16><<<grid, 256, 0, s>>>(g); break;
    case HMX_EPI_SILU: gemm_bf16_dma_kernel<LB, ACT_SILU, BF16><<<grid, 256, 0, s>>>(g); break;
    default: gemm_bf16_dma_kernel<LB, ACT_ID, BF16><<<grid, 256, 0, s>>>(g); break;
  }
}

template <int LB>
void launch_bf16_dma_b(const GemmArgs& g, dim3 grid, hipStream_t s) {
  if (g.c_dtype == HMX_DTYPE_BF16)
    launch_bf16_dma_c<LB, true>(g, grid, s);
  else
    launch_bf16_dma_c<LB, false>(g, grid, s);
}

void launch_bf16_dma(const GemmArgs& g, int lb, dim3 grid, hipStream_t s) {
  if (lb == L_RCONTIG)
    launch_bf16_dma_b<L_RCONTIG>(g, grid, s);
  else
    launch_bf16_dma_b<L_KCONTIG>(g, grid, s);
}

template <class Cfg, int LA, int LB>
void launch_f32(const GemmArgs& g, bool guard, dim3 grid, hipStream_t s) {
  if (guard)
    gemm_f32_kernel<Cfg, LA, LB, true><<<grid, Cfg::NT, 0, s>>>(g);
  else
    gemm_f32_kernel<Cfg, LA, LB, false><<<grid, Cfg::NT, 0, s>>>(g);
}

template <class Cfg>
void dispatch_f32(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s) {
  if constexpr (Cfg::BM == 256) {
    if (lb == L_RCONTIG)
      launch_f32<Cfg, L_KCONTIG, L_RCONTIG>(g, guard, grid, s);
    else
      launch_f32<Cfg, L_KCONTIG, L_KCONTIG>(g, guard, grid, s);
  } else if (la == L_KCONTIG) {
    switch (lb) {
      case L_KCONTIG: launch_f32<Cfg, L_KCONTIG, L_KCONTIG>(g, guard, grid, s); break;
      case L_RCONTIG: launch_f32<Cfg, L_KCONTIG, L_RCONTIG>(g, guard, grid, s); break;
      case L_BLOCKED: launch_f32<Cfg, L_KCONTIG, L_BLOCKED>(g, guard, grid, s); break;
      case L_PANELS: launch_f32<Cfg, L_KCONTIG, L_PANELS>(g, guard, grid, s); break;
    }
  } else {
    if (lb == L_KCONTIG)
      launch_f32<Cfg, L_RCONTIG, L_KCONTIG>(g, guard, grid, s);
    else
      launch_f32<Cfg, L_RCONTIG, L_RCONTIG>(g, guard, grid, s);
  }
}

}  // namespace
}  // namespace hmx

using namespace hmx;

extern "C" {

int hmx_gemm_plan(int ab_dtype, int64_t m, int64_t n, int64_t k, int64_t batch, int trans_a,
                  int b_layout, int splits, int64_t max_workspace_bytes, int tile_m,
                  int tile_n, int tile_k, int* out_splits, int* out_tile_m, int* out_tile_n,
                  int* out_tile_k, int64_t* out_workspace_bytes) {
  HMX_REQUIRE(valid_dtype(ab_dtype), "gemm_plan: unknown dtype %d", ab_dtype);
  HMX_REQUIRE(layout_code(b_layout) >= 0, "gemm_plan: unknown B layout %d", b_layout);
  HMX_REQUIRE(m >= 0 && n >= 0 && k >= 0 && batch >= 1, "gemm_plan: invalid shape");
  HMX_REQUIRE(splits >= 0, "gemm_plan: negative splits");
  Plan plan;
  int st = make_plan(ab_dtype, m, n, k, batch, trans_a, b_layout, splits, max_workspace_bytes, tile_m,
                     tile_n, tile_k, plan);
  if (st != HMX_OK) return st;
  if (out_splits) *out_splits = plan.splits;
  if (out_tile_m) *out_tile_m = plan.tile.bm;
  if (out_tile_n) *out_tile_n = plan.tile.bn;
  if (out_tile_k) *out_tile_k = plan.tile.bk;
  if (out_workspace_bytes) *out_workspace_bytes = plan.workspace_bytes;
  return HMX_OK;
}

int hmx_gemm(int ab_dtype, int c_dtype, const void* a, int64_t lda, int trans_a,
             const void* b, int64_t ldb, int b_layout, int64_t b_panel, int64_t b_kpad,
             void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t batch,
             int64_t stride_a, int64_t stride_b, int64_t stride_c, const void* bias,
             const void* scale, const void* shift, int vec_dtype, int epilogue,
             float epilogue_arg, int splits, void* workspace, int64_t workspace_bytes,
             int tile_m, int tile_n, int tile_k, void* stream) {
  HMX_REQUIRE(valid_dtype(ab_dtype) && valid_dtype(c_dtype), "gemm: unknown dtype");
  HMX_REQUIRE((bias == nullptr && scale == nullptr && shift == nullptr) || valid_dtype(vec_dtype),
              "gemm: unknown vector dtype %d", vec_dtype);
  HMX_REQUIRE(valid_activation(epilogue), "gemm: unknown epilogue %d", epilogue);
  const int lb = layout_code(b_layout);
  HMX_REQUIRE(lb >= 0, "gemm: unknown B layout %d", b_layout);
  HMX_REQUIRE(ab_dtype == HMX_DTYPE_BF16 || lb == L_KCONTIG || lb == L_RCONTIG ||
                  lb == L_BLOCKED || lb == L_PANELS,
              "gemm: VNNI layouts pair bf16 values; f32 B takes row-major, blocked or panel layouts");
  HMX_REQUIRE(!trans_a || lb == L_KCONTIG || lb == L_RCONTIG,
              "gemm: packed B layouts take a row-major A");
  HMX_REQUIRE(m >= 0 && n >= 0 && k >= 0 && batch >= 1, "gemm: invalid shape [%lld, %lld, %lld] x %lld",
              (long long)m, (long long)n, (long long)k, (long long)batch);
  HMX_REQUIRE(a && b && c, "gemm: null operand");
  HMX_REQUIRE(splits >= 0, "gemm: negative splits");
  const bool packed = lb != L_KCONTIG && lb != L_RCONTIG;
  if (!packed) {
    HMX_REQUIRE(lda >= (trans_a ? m : k) && lda >= 1, "gemm: lda %lld too small", (long long)lda);
    HMX_REQUIRE(ldb >= (lb == L_KCONTIG ? k : n) && ldb >= 1, "gemm: ldb %lld too small", (long long)ldb);
  } else {
    HMX_REQUIRE(b_kpad >= k && b_kpad % (lb == L_VNNI_PANELS ? 2 : 1) == 0,
                "gemm: packed K extent %lld does not cover K %lld", (long long)b_kpad, (long long)k);
    if (lb == L_BLOCKED_VNNI || lb == L_BLOCKED)
      HMX_REQUIRE(b_kpad % 32 == 0, "gemm: blocked K extent %lld is not a multiple of 32", (long long)b_kpad);
    if (lb == L_VNNI_PANELS || lb == L_PANELS)
      HMX_REQUIRE(b_panel >= 8 && b_panel % (lb == L_VNNI_PANELS ? 4 : 8) == 0,
                  "gemm: panel width %lld unsupported", (long long)b_panel);
  }
  HMX_REQUIRE(ldc >= n && ldc >= 1, "gemm: ldc %lld too small", (long long)ldc);
  if (m == 0 || n == 0) return HMX_OK;

  Plan plan;
  make_plan(ab_dtype, m, n, k, batch, trans_a, b_layout, splits, workspace ? workspace_bytes : 0,
            tile_m, tile_n, tile_k, plan);
  if (plan.splits > 1) {
    HMX_REQUIRE(workspace != nullptr && workspace_bytes >= plan.workspace_bytes,
                "gemm: split-K needs %lld workspace bytes, got %lld",
                (long long)plan.workspace_bytes, (long long)workspace_bytes);
  }
  void* partials = workspace ? (char*)workspace + plan.bt_bytes : nullptr;
  int lb_run = lb;
  if (plan.transpose_b) {
    // B [K, N] -> B^T [N, K] in the workspace; the GEMM then reads it K-contiguous.
    launch_transpose16(b, workspace, k, n, ldb, (hipStream_t)stream);
    const int st = check_launch("gemm B transpose");
    if (st != HMX_OK) return st;
    b = workspace;
    ldb = k;
    lb_run = L_KCONTIG;
  }
  const int64_t tiles_m = ceil_div(m, plan.tile.bm), tiles_n = ceil_div(n, plan.tile.bn);
  HMX_REQUIRE(tiles_m * tiles_n < ((int64_t)1 << 31) && batch < 65536 && plan.splits < 65536,
              "gemm: grid too large");

  const int64_t esz = dtype_bytes(ab_dtype);
  const int64_t vec_elems = 16 / esz;
  GemmArgs g{};
  const int la = trans_a ? L_RCONTIG : L_KCONTIG;
  g.a = Operand{a, lda, m, 0, 0,
                aligned16(a) && lda % vec_elems == 0 && (batch == 1 || stride_a % vec_elems == 0), 0};
  const int64_t b_rows = packed ? (lb == L_BLOCKED_VNNI || lb == L_BLOCKED ? ceil_div(n, 32) * 32
                                                                           : ceil_div(n, b_panel) * b_panel)
                                : n;
  g.b = Operand{b, ldb, b_rows, b_panel, b_kpad,
                aligned16(b) && (packed || ldb % vec_elems == 0) &&
                    (batch == 1 || stride_b % vec_elems == 0),
                0};
  // Bytes spanned by one batch slice of each operand: the buffer-load
  // range of the whole-tile path, which needs it below 2^31.
  const int64_t a_bytes = (trans_a ? (k - 1) * lda + m : (m - 1) * lda + k) * esz;
  const int64_t b_bytes =
      packed ? b_rows * b_kpad * esz : (lb_run == L_RCONTIG ? (k - 1) * ldb + n : (n - 1) * ldb + k) * esz;
  const bool bytes_ok = a_bytes < INT32_MAX && b_bytes < INT32_MAX;
  g.a.bytes = bytes_ok ? (int32_t)a_bytes : 0;
  g.b.bytes = bytes_ok ? (int32_t)b_bytes : 0;
  // Packed layouts read zeros (their padding) past N up to the padded extent;
  // columns past N are never stored.
  g.stride_a = stride_a;
  g.stride_b = stride_b;
  g.m = m;
  g.n = n;
  g.k = k;
  g.k_chunk = plan.k_chunk;
  g.tiles_m = (int)tiles_m;
  g.tiles_n = (int)tiles_n;
  g.bias = bias;
  g.scale = scale;
  g.shift = shift;
  g.vec_dtype = vec_dtype;
  g.act = epilogue;
  g.act_arg = epilogue_arg;
  if (plan.splits > 1) {
    g.c = partials;
    g.c_dtype = HMX_DTYPE_F32;
    g.ldc = n;
    g.stride_c = m * n;
    g.stride_split = batch * m * n;
    g.bias = g.scale = g.shift = nullptr;
    g.act = HMX_EPI_IDENTITY;
  } else {
    g.c = c;
    g.c_dtype = c_dtype;
    g.ldc = ldc;
    g.stride_c = stride_c;
    g.stride_split = 0;
  }

  const bool whole = m % plan.tile.bm == 0 && n % plan.tile.bn == 0 &&
                     plan.k_chunk % plan.tile.bk == 0 && k % plan.tile.bk == 0;
  const bool guard = !(whole && g.a.vec && g.b.vec && bytes_ok);
  const dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)plan.splits, (unsigned)batch);
  auto s = (hipStream_t)stream;
  if (ab_dtype == HMX_DTYPE_BF16) {
    const TileChoice t = plan.tile;
    if (t.bm == 256 && !guard && la == L_KCONTIG && (lb_run == L_KCONTIG || lb_run == L_RCONTIG) &&
        dma_direct_ok(g) && dma_enabled())
      launch_bf16_dma(g, lb_run, grid, s);
    else if (t.bm == 256)
      dispatch_bf16<Bf16Cfg<256, 256, 64>>(g, la, lb_run, guard, grid, s);
    else
      dispatch_bf16<Bf16Cfg<128, 128, 64>>(g, la, lb_run, guard, grid, s);
  } else if (plan.tile.bm == 256) {
    // Planned only for row-major A, B [N, K] or [K, N] and two or more
    // splits, so the kernel writes f32 partials with the identity epilogue.
    if (plan.splits < 2 || la != L_KCONTIG)
      return set_error(HMX_ERR_INVALID, "gemm: internal f32 plan without split-K");
    dispatch_f32<F32Cfg<256, 256, 16>>(g, la, lb, guard, grid, s);
  } else {
    dispatch_f32<F32Cfg<128, 128, 32>>(g, la, lb, guard, grid, s);
  }
  int st = check_launch("gemm");
  if (st != HMX_OK || plan.splits <= 1) return st;

  GemmArgs r = g;
  r.c = c;
  r.c_dtype = c_dtype;
  r.ldc = ldc;
  r.stride_c = stride_c;
  r.bias = bias;
  r.scale = scale;
  r.shift = shift;
  r.act = epilogue;
  const int64_t total = batch * m * n;
  const int64_t c_align = c_dtype == HMX_DTYPE_BF16 ? 8 : 16;
  const bool vec4 = n % 4 == 0 && ldc % 4 == 0 && stride_c % 4 == 0 && ((uintptr_t)c % c_align) == 0 &&
                    ((uintptr_t)partials % 16) == 0;
  if (vec4) {
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(total / 4, 256), 16384);
    splitk_reduce_kernel<4><<<blocks, 256, 0, s>>>((const float*)partials, plan.splits, batch, r);
  } else {
    const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(total, 256), 16384);
    splitk_reduce_kernel<1><<<blocks, 256, 0, s>>>((const float*)partials, plan.splits, batch, r);
  }
  return check_launch("gemm split-K reduce");
}

}  // extern "C"
