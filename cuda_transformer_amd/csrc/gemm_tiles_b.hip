// GEMM kernel instances of the narrow and narrow192 tiles (kernels: gemm_kernel.hpp).  The tile
// types are spread over three files so that the build compiles them in parallel.
#include "gemm_kernel.hpp"

namespace cta {

int gemm_launch_narrow(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                       const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                       int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats) {
  return gemm_launch_tile<NarrowTile>(A, B, C, ep, M, N, K, Z, zin, st, workspace,
                                       workspace_floats);
}

int gemm_launch_narrow192(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                          const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                          int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats) {
  return gemm_launch_tile<Narrow192Tile>(A, B, C, ep, M, N, K, Z, zin, st, workspace,
                                          workspace_floats);
}

}  // namespace cta
