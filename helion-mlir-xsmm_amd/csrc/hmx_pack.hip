// Layout conversion kernels for gfx950: zero padding and the blocked, VNNI
// and panel packings of GEMM operands.
//
// Every kind is a gather: one thread per destination element computes the
// logical element (i, j) it holds and reads it from the source (zero past the
// source's extent), so destination writes are fully coalesced. The logical
// matrix L is the source or, for the *_T kinds, its transpose.
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
  const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(a.total, 256), 65536);
  if (dtype == HMX_DTYPE_BF16)
    launch(pack_kernel<uint16_t>, blocks, 256, s, a);
  else
    launch(pack_kernel<float>, blocks, 256, s, a);
  return check_launch("pack");
}
