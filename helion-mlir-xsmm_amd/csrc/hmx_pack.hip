// Layout conversion kernels for gfx950: zero padding and the blocked, VNNI
// and panel packings of GEMM operands.
//
// The logical matrix L is the source or, for the *_T kinds, its transpose.
// Every kind runs as 64 x 64 tiles of L staged through LDS (pack_tiled_kernel)
// and written in 16-byte destination runs; VNNI panels of a transposed weight
// with panels of a multiple of 64 columns take a word-transpose kernel; a
// one-element-per-thread gather (pack_kernel) remains for grids too tall for
// the tiles.
#include "hmx_device.hpp"

namespace hmx {
namespace {

struct PackArgs {
  const void* src;
  void* dst;
  int64_t rows, cols, ld;        // source as stored
  int64_t lrows, lcols;          // extent of L
  int64_t rows_pad, cols_pad;    // padded extent of L
  int64_t panel;
  int64_t total;
  int kind;
  bool transposed;
};

// Logical (i, j) of destination element d.
__device__ __forceinline__ void dst_coords(const PackArgs& a, int64_t d, int64_t& i, int64_t& j) {
  const int64_t rp = a.rows_pad, cp = a.cols_pad;
  switch (a.kind) {
    case HMX_PACK_A_BLOCKED:
    case HMX_PACK_A_BLOCKED_T: {  // [RP/32][CP/32][32][32]
      const int64_t jj = d & 31, ii = (d >> 5) & 31, blk = d >> 10;
      const int64_t jb = blk % (cp >> 5), ib = blk / (cp >> 5);
      i = ib * 32 + ii;
      j = jb * 32 + jj;
      return;
    }
    case HMX_PACK_B_BLOCKED:
    case HMX_PACK_B_BLOCKED_T: {  // [CP/32][RP/32][32][32], block [k][n]
      const int64_t jj = d & 31, ii = (d >> 5) & 31, blk = d >> 10;
      const int64_t kb = blk % (rp >> 5), nb = blk / (rp >> 5);
      i = kb * 32 + ii;
      j = nb * 32 + jj;
      return;
    }
    case HMX_PACK_B_BLOCKED_VNNI:
    case HMX_PACK_B_BLOCKED_VNNI_T: {  // [CP/32][RP/32][16][32][2]
      const int64_t p = d & 1, n = (d >> 1) & 31, r = (d >> 6) & 15, blk = d >> 10;
      const int64_t kb = blk % (rp >> 5), nb = blk / (rp >> 5);
      i = kb * 32 + 2 * r + p;
      j = nb * 32 + n;
      return;
    }
    case HMX_PACK_B_VNNI_PANELS_T: {  // [CP/P][RP/2][P][2]
      const int64_t p = d & 1, rest = d >> 1;
      const int64_t n = rest % a.panel, rest2 = rest / a.panel;
      const int64_t c = rest2 % (rp >> 1), jp = rest2 / (rp >> 1);
      i = 2 * c + p;
      j = jp * a.panel + n;
      return;
    }
    case HMX_PACK_B_PANELS: {  // [CP/P][RP][P]
      const int64_t n = d % a.panel, rest = d / a.panel;
      const int64_t k = rest % rp, jp = rest / rp;
      i = k;
      j = jp * a.panel + n;
      return;
    }
    case HMX_PACK_A_PANELS: {  // [CP/P][RP][P]
      const int64_t t = d % a.panel, rest = d / a.panel;
      const int64_t m = rest % rp, kb = rest / rp;
      i = m;
      j = kb * a.panel + t;
      return;
    }
    default: {  // HMX_PACK_PAD: [RP][CP]
      i = d / cp;
      j = d % cp;
      return;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(PackArgs a) {
  const T* src = (const T*)a.src;
  T* dst = (T*)a.dst;
  for (int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; d < a.total;
       d += (int64_t)gridDim.x * blockDim.x) {
    int64_t i, j;
    dst_coords(a, d, i, j);
    T v = T(0);
    if (i < a.lrows && j < a.lcols) v = src[a.transposed ? j * a.ld + i : i * a.ld + j];
    dst[d] = v;
  }
}

// Destination index of logical element (i, j): the inverse of dst_coords.
__device__ __forceinline__ int64_t dst_index(const PackArgs& a, int64_t i, int64_t j) {
  const int64_t rp = a.rows_pad, cp = a.cols_pad, pn = a.panel;
  switch (a.kind) {
    case HMX_PACK_A_BLOCKED:
    case HMX_PACK_A_BLOCKED_T:
      return (((i >> 5) * (cp >> 5) + (j >> 5)) * 32 + (i & 31)) * 32 + (j & 31);
    case HMX_PACK_B_BLOCKED:
    case HMX_PACK_B_BLOCKED_T:
      return (((j >> 5) * (rp >> 5) + (i >> 5)) * 32 + (i & 31)) * 32 + (j & 31);
    case HMX_PACK_B_BLOCKED_VNNI:
    case HMX_PACK_B_BLOCKED_VNNI_T:
      return (((((j >> 5) * (rp >> 5) + (i >> 5)) * 16 + ((i & 31) >> 1)) * 32 + (j & 31)) * 2) + (i & 1);
    case HMX_PACK_B_VNNI_PANELS_T:
      return (((j / pn) * (rp >> 1) + (i >> 1)) * pn + (j % pn)) * 2 + (i & 1);
    case HMX_PACK_B_PANELS:
    case HMX_PACK_A_PANELS:
      return ((j / pn) * rp + i) * pn + (j % pn);
    default:  // PAD, TRANSPOSE: [RP][CP]
      return i * cp + j;
  }
}

// Columns per destination run that stay contiguous: the 32-wide blocks, the
// panel, or the whole padded row.
__device__ __forceinline__ bool run_contiguous(const PackArgs& a, int64_t j, int len) {
  switch (a.kind) {
    case HMX_PACK_B_VNNI_PANELS_T:
    case HMX_PACK_B_PANELS:
    case HMX_PACK_A_PANELS:
      return (j % a.panel) + len <= a.panel;
    case HMX_PACK_PAD:
    case HMX_PACK_TRANSPOSE:
      return true;
    default:
      return (j & 31) + len <= 32;
  }
}

__device__ __forceinline__ bool vnni_kind(int kind) {
  return kind == HMX_PACK_B_BLOCKED_VNNI || kind == HMX_PACK_B_BLOCKED_VNNI_T ||
         kind == HMX_PACK_B_VNNI_PANELS_T;
}

// Eight consecutive elements of stored row `r` from column `c` (zero outside
// [rows, cols)): 16-byte loads when `vec` (16-byte aligned base and lines).
template <typename T>
__device__ __forceinline__ void load8(const T* __restrict__ src, int64_t ld, int64_t r, int64_t c,
                                      int64_t rows, int64_t cols, bool vec, T (&v)[8]) {
  if (vec && r < rows && c + 8 <= cols) {
    const uint4* p = (const uint4*)(src + r * ld + c);
#pragma unroll
    for (int h = 0; h < (int)sizeof(T) * 8 / 16; ++h) {
      const uint4 u = p[h];
      __builtin_memcpy(&v[h * (16 / (int)sizeof(T))], &u, 16);
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (r < rows && c + e < cols) ? src[r * ld + c + e] : T(0);
}

// Every layout of the pack kinds in one tiled kernel: workgroup (bx, by)
// loads the 64 x 64 tile of the padded logical matrix L at (64 by, 64 bx)
// into LDS (16-byte row loads; a transposed source is read along its own
// rows and stored transposed), then writes it as runs of 8 destination
// elements with 16-byte stores: 8 consecutive columns of one row, or, for the
// VNNI layouts, 4 columns of a row pair (K pairs are innermost). Runs that
// leave the padded extent, a block or a panel, or 16-byte alignment, are
// written element by element. Zero past the source's extent.
template <typename T>
__global__ __launch_bounds__(256) void pack_tiled_kernel(PackArgs a, bool vec_src, bool vec_dst) {
  constexpr int TL = 64, PITCH = TL + 8;
  __shared__ T tile[TL * PITCH];
  const T* src = (const T*)a.src;
  T* dst = (T*)a.dst;
  const int64_t i0 = (int64_t)blockIdx.y * TL, j0 = (int64_t)blockIdx.x * TL;
  const int t = threadIdx.x;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int rl = (t >> 3) + 32 * pass, cl = (t & 7) * 8;
    T v[8];
    if (!a.transposed) {
      load8<T>(src, a.ld, i0 + rl, j0 + cl, a.lrows, a.lcols, vec_src, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) tile[rl * PITCH + cl + e] = v[e];
    } else {
      // Stored row j0 + rl holds L's column j0 + rl; its columns are L's rows.
      load8<T>(src, a.ld, j0 + rl, i0 + cl, a.lcols, a.lrows, vec_src, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) tile[(cl + e) * PITCH + rl] = v[e];
    }
  }
  __syncthreads();
  constexpr int VE = 16 / (int)sizeof(T);  // elements per 16-byte store
  if (vnni_kind(a.kind)) {
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int pl = (t >> 4) + 16 * pass, jl = (t & 15) * 4;  // row pair, 4 columns
      const int64_t i = i0 + 2 * pl, j = j0 + jl;
      if (i >= a.rows_pad) continue;
      const int64_t d = dst_index(a, i, j);
      if (vec_dst && i + 1 < a.rows_pad && j + 4 <= a.cols_pad && run_contiguous(a, j, 4) && d % VE == 0) {
        T v[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[2 * q] = tile[(2 * pl) * PITCH + jl + q];
          v[2 * q + 1] = tile[(2 * pl + 1) * PITCH + jl + q];
        }
#pragma unroll
        for (int h = 0; h < 8 / VE; ++h) {
          uint4 u;
          __builtin_memcpy(&u, &v[h * VE], 16);
          *(uint4*)(dst + d + h * VE) = u;
        }
      } else {
        for (int p = 0; p < 2; ++p)
          for (int q = 0; q < 4; ++q)
            if (i + p < a.rows_pad && j + q < a.cols_pad)
              dst[dst_index(a, i + p, j + q)] = tile[(2 * pl + p) * PITCH + jl + q];
      }
    }
  } else {
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int rl = (t >> 3) + 32 * pass, cl = (t & 7) * 8;
      const int64_t i = i0 + rl, j = j0 + cl;
      if (i >= a.rows_pad) continue;
      const int64_t d = dst_index(a, i, j);
      if (vec_dst && j + 8 <= a.cols_pad && run_contiguous(a, j, 8) && d % VE == 0) {
#pragma unroll
        for (int h = 0; h < 8 / VE; ++h) {
          uint4 u;
          __builtin_memcpy(&u, &tile[rl * PITCH + cl + h * VE], 16);
          *(uint4*)(dst + d + h * VE) = u;
        }
      } else {
        for (int e = 0; e < 8; ++e)
          if (j + e < a.cols_pad) dst[dst_index(a, i, j + e)] = tile[rl * PITCH + cl + e];
      }
    }
  }
}

// VNNI panels of a transposed bf16 weight W [N, K] (row stride ld, K even):
// dst[jp][c][n] (32-bit words, [N_pad/P][K_pad/2][P]) = the K pair
// (W[jp P + n][2c], W[jp P + n][2c + 1]), zero past N and K. Viewing W's rows
// as words, a panel is the transpose of a [P, K/2] word matrix, so each
// workgroup transposes a 64 x 64 word tile through LDS: each load (store)
// instruction has 16 threads cover one row's 256 bytes, 16 rows per pass,
// four passes (P a multiple of 64: a tile's columns stay in one panel).
// VEC: rows keep 16-byte alignment (ld % 8 == 0, 16-byte aligned W).
template <bool VEC>
__global__ __launch_bounds__(256) void pack_vnni_t_kernel(const uint16_t* __restrict__ w,
                                                          uint32_t* __restrict__ dst, int64_t n_rows,
                                                          int64_t k, int64_t ld, int64_t kp_words,
                                                          int64_t panel) {
  constexpr int PITCH = 65;
  __shared__ uint32_t tile[64 * PITCH];
  const int t = threadIdx.x, q4 = (t & 15) * 4;
  const int64_t n0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int64_t kw = k / 2;  // words per source row
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int nl = pass * 16 + (t >> 4);
    const int64_t n = n0 + nl, c = c0 + q4;
    const uint32_t* row = (const uint32_t*)(w + n * ld);
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    if (n < n_rows) {
      if (VEC && c + 4 <= kw) {
        const uint4 u = *(const uint4*)(row + c);
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < kw) v[e] = row[c + e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[nl * PITCH + q4 + e] = v[e];
  }
  __syncthreads();
  const int64_t jp = n0 / panel;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int cl = pass * 16 + (t >> 4);
    const int64_t c = c0 + cl;
    if (c < kp_words) {
      uint4 u;
      u.x = tile[q4 * PITCH + cl];
      u.y = tile[(q4 + 1) * PITCH + cl];
      u.z = tile[(q4 + 2) * PITCH + cl];
      u.w = tile[(q4 + 3) * PITCH + cl];
      *(uint4*)(dst + (jp * kp_words + c) * panel + (n0 % panel) + q4) = u;
    }
  }
}

// Transpose of 16-bit elements, [rows, cols] (row stride ld) -> [cols, rows]
// contiguous. Each lane moves an 8 x 8 block: eight 16-byte row loads, a
// register transpose (v_perm_b32), eight 16-byte stores; a wave covers a
// 64 x 64 tile with 128-byte segments on both sides. Edge blocks go element
// by element.
__device__ __forceinline__ uint32_t lo_pair(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}
__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ src,
                                                          uint16_t* __restrict__ dst, int64_t rows,
                                                          int64_t cols, int64_t ld, bool vec) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.y * 64 + (lane & 7) * 8;
  const int64_t c0 = ((int64_t)blockIdx.x * 4 + wave) * 64 + (lane >> 3) * 8;
  if (r0 >= rows || c0 >= cols) return;
  uint4 in[8];
  const bool whole = vec && r0 + 8 <= rows && c0 + 8 <= cols;
  if (whole) {
#pragma unroll
    for (int k = 0; k < 8; ++k) in[k] = *(const uint4*)(src + (r0 + k) * ld + c0);
    // Output row j (source column c0 + j) holds source rows r0..r0+7.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint4 o;
      const int d = j >> 1;
      if (j & 1) {
        o = make_uint4(hi_pair(word(in[0], d), word(in[1], d)), hi_pair(word(in[2], d), word(in[3], d)),
                       hi_pair(word(in[4], d), word(in[5], d)), hi_pair(word(in[6], d), word(in[7], d)));
      } else {
        o = make_uint4(lo_pair(word(in[0], d), word(in[1], d)), lo_pair(word(in[2], d), word(in[3], d)),
                       lo_pair(word(in[4], d), word(in[5], d)), lo_pair(word(in[6], d), word(in[7], d)));
      }
      *(uint4*)(dst + (c0 + j) * rows + r0) = o;
    }
  } else {
    for (int j = 0; j < 8 && c0 + j < cols; ++j)
      for (int k = 0; k < 8 && r0 + k < rows; ++k) dst[(c0 + j) * rows + r0 + k] = src[(r0 + k) * ld + c0 + j];
  }
}

constexpr int64_t kMaxGridX = 0x7fffffff;

bool is_transposed(int kind) {
  return kind == HMX_PACK_A_BLOCKED_T || kind == HMX_PACK_B_BLOCKED_T ||
         kind == HMX_PACK_B_BLOCKED_VNNI_T || kind == HMX_PACK_B_VNNI_PANELS_T ||
         kind == HMX_PACK_TRANSPOSE;
}

}  // namespace

void launch_transpose16(const void* src, void* dst, int64_t rows, int64_t cols, int64_t ld,
                        hipStream_t stream) {
  const bool vec = aligned16(src) && aligned16(dst) && ld % 8 == 0 && rows % 8 == 0;
  const dim3 grid((unsigned)ceil_div(cols, 256), (unsigned)ceil_div(rows, 64));
  launch(transpose16_kernel, grid, 256, stream, (const uint16_t*)src, (uint16_t*)dst, rows, cols,
         ld, vec);
}

}  // namespace hmx

using namespace hmx;

extern "C" int hmx_pack(int kind, int dtype, const void* src, int64_t rows, int64_t cols,
                        int64_t ld, void* dst, int64_t rows_pad, int64_t cols_pad,
                        int64_t panel, void* stream) {
  HMX_REQUIRE(valid_dtype(dtype), "pack: unknown dtype %d", dtype);
  HMX_REQUIRE(kind >= HMX_PACK_PAD && kind <= HMX_PACK_TRANSPOSE, "pack: unknown kind %d", kind);
  HMX_REQUIRE(rows >= 0 && cols >= 0 && rows_pad >= 0 && cols_pad >= 0, "pack: invalid shape");
  HMX_REQUIRE(src && dst, "pack: null operand");
  HMX_REQUIRE(ld >= cols, "pack: ld %lld smaller than %lld columns", (long long)ld, (long long)cols);
  const bool t = is_transposed(kind);
  const int64_t lrows = t ? cols : rows, lcols = t ? rows : cols;
  HMX_REQUIRE(rows_pad >= lrows && cols_pad >= lcols, "pack: padded extent smaller than the matrix");
  switch (kind) {
    case HMX_PACK_A_BLOCKED:
    case HMX_PACK_A_BLOCKED_T:
    case HMX_PACK_B_BLOCKED:
    case HMX_PACK_B_BLOCKED_T:
    case HMX_PACK_B_BLOCKED_VNNI:
    case HMX_PACK_B_BLOCKED_VNNI_T:
      HMX_REQUIRE(rows_pad % 32 == 0 && cols_pad % 32 == 0,
                  "pack: blocked extents must be multiples of 32");
      break;
    case HMX_PACK_B_VNNI_PANELS_T:
      HMX_REQUIRE(panel >= 1 && cols_pad % panel == 0 && rows_pad % 2 == 0,
                  "pack: VNNI panels need N_pad %% panel == 0 and an even K_pad");
      break;
    case HMX_PACK_B_PANELS:
    case HMX_PACK_A_PANELS:
      HMX_REQUIRE(panel >= 1 && cols_pad % panel == 0, "pack: panel must divide the columns");
      break;
    default:
      break;
  }
  PackArgs a{src, dst, rows, cols, ld, lrows, lcols, rows_pad, cols_pad, panel,
             rows_pad * cols_pad, kind, t};
  if (a.total == 0) return HMX_OK;
  auto s = (hipStream_t)stream;
  if (kind == HMX_PACK_TRANSPOSE && dtype == HMX_DTYPE_BF16 && rows_pad == lrows &&
      cols_pad == lcols && rows > 0 && cols > 0) {
    launch_transpose16(src, dst, rows, cols, ld, s);
    return check_launch("pack transpose");
  }
  if (kind == HMX_PACK_B_VNNI_PANELS_T && dtype == HMX_DTYPE_BF16 && panel % 64 == 0 && rows > 0 &&
      cols % 2 == 0 && ld % 2 == 0 && ((uintptr_t)src & 3) == 0 && aligned16(dst) &&
      ceil_div(rows_pad / 2, 64) <= 65535) {
    // rows = N, cols = K of the stored W; rows_pad = K_pad, cols_pad = N_pad.
    const dim3 grid((unsigned)(cols_pad / 64), (unsigned)ceil_div(rows_pad / 2, 64));
    const bool vec = ld % 8 == 0 && aligned16(src);
    if (vec)
      launch(pack_vnni_t_kernel<true>, grid, 256, s, (const uint16_t*)src, (uint32_t*)dst, rows, cols, ld,
             rows_pad / 2, panel);
    else
      launch(pack_vnni_t_kernel<false>, grid, 256, s, (const uint16_t*)src, (uint32_t*)dst, rows, cols, ld,
             rows_pad / 2, panel);
    return check_launch("pack VNNI panels");
  }
  if (ceil_div(rows_pad, 64) <= 65535 && ceil_div(cols_pad, 64) <= kMaxGridX) {
    const int64_t esz = dtype_bytes(dtype);
    const bool vec_src = aligned16(src) && ld % (16 / esz) == 0;
    const dim3 grid((unsigned)ceil_div(cols_pad, 64), (unsigned)ceil_div(rows_pad, 64));
    if (dtype == HMX_DTYPE_BF16)
      launch(pack_tiled_kernel<uint16_t>, grid, 256, s, a, vec_src, aligned16(dst));
    else
      launch(pack_tiled_kernel<float>, grid, 256, s, a, vec_src, aligned16(dst));
    return check_launch("pack");
  }
  const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(a.total, 256), 65536);
  if (dtype == HMX_DTYPE_BF16)
    launch(pack_kernel<uint16_t>, blocks, 256, s, a);
  else
    launch(pack_kernel<float>, blocks, 256, s, a);
  return check_launch("pack");
}
