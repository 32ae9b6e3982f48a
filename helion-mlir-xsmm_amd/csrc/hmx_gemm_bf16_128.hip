// The register-staged bf16 GEMM kernel at 128 x 128 tiles (shapes whose
// 256 x 256 tiles would underfill the GPU), row-major or transposed A and B.
#include "hmx_gemm_bf16.hpp"

namespace hmx {

void launch_gemm_bf16_128(const GemmArgs& g, int la, int lb, bool guard, dim3 grid, hipStream_t s) {
  dispatch_bf16_plain<Bf16Cfg<128, 128, 64>>(g, la, lb, guard, grid, s);
}

}  // namespace hmx
