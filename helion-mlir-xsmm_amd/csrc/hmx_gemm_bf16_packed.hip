// The register-staged bf16 GEMM kernel reading a packed B in place (VNNI
// panels, VNNI blocks, bench panels, 32 x 32 blocks) at 256 x 256 tiles; A is
// row-major.
#include "hmx_gemm_bf16.hpp"

namespace hmx {

void launch_gemm_bf16_packed(const GemmArgs& g, int lb, bool guard, dim3 grid, hipStream_t s) {
  using Cfg = Bf16Cfg<256, 256, 64>;
  switch (lb) {
    case L_VNNI_PANELS: launch_bf16<Cfg, L_KCONTIG, L_VNNI_PANELS>(g, guard, grid, s); break;
    case L_BLOCKED_VNNI: launch_bf16<Cfg, L_KCONTIG, L_BLOCKED_VNNI>(g, guard, grid, s); break;
    case L_PANELS: launch_bf16<Cfg, L_KCONTIG, L_PANELS>(g, guard, grid, s); break;
    case L_BLOCKED: launch_bf16<Cfg, L_KCONTIG, L_BLOCKED>(g, guard, grid, s); break;
  }
}

}  // namespace hmx
