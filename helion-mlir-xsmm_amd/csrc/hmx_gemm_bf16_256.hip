// The register-staged bf16 GEMM kernel at 256 x 256 tiles, row-major or
// transposed A and B; and the bf16 launcher that picks among the units.
#include "hmx_gemm_bf16.hpp"

namespace hmx {

void launch_gemm_bf16_256(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s) {
  dispatch_bf16_plain<Bf16Cfg<256, 256, 64>>(g, la, lb, guard, grid, s);
}

void launch_gemm_bf16(const GemmArgs& g, int tile_bm, int la, int lb, bool guard, dim3 grid,
                      hipStream_t s) {
  const bool plain = (la == L_KCONTIG || la == L_RCONTIG) && (lb == L_KCONTIG || lb == L_RCONTIG);
  if (!plain)
    launch_gemm_bf16_packed(g, lb, guard, grid, s);  // packed B: 256 x 256 tiles, A K-contiguous
  else if (tile_bm == 256)
    launch_gemm_bf16_256(g, la, lb, guard, grid, s);
  else
    launch_gemm_bf16_128(g, la, lb, guard, grid, s);
}

}  // namespace hmx
