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

bool is_transposed(int kind) {
  return kind == HMX_PACK_A_BLOCKED_T || kind == HMX_PACK_B_BLOCKED_T ||
         kind == HMX_PACK_B_BLOCKED_VNNI_T || kind == HMX_PACK_B_VNNI_PANELS_T;
}

}  // namespace
}  // namespace hmx

using namespace hmx;

extern "C" int hmx_pack(int kind, int dtype, const void* src, int64_t rows, int64_t cols,
                        int64_t ld, void* dst, int64_t rows_pad, int64_t cols_pad,
                        int64_t panel, void* stream) {
  HMX_REQUIRE(valid_dtype(dtype), "pack: unknown dtype %d", dtype);
  HMX_REQUIRE(kind >= HMX_PACK_PAD && kind <= HMX_PACK_A_PANELS, "pack: unknown kind %d", kind);
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
  const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(a.total, 256), 65536);
  if (dtype == HMX_DTYPE_BF16)
    pack_kernel<uint16_t><<<blocks, 256, 0, s>>>(a);
  else
    pack_kernel<float><<<blocks, 256, 0, s>>>(a);
  return check_launch("pack");
}
