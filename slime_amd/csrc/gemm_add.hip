// gemm_add.hip — the backward's dX GEMM with its epilogue adding the direct part:
// grad_x = gXd + [gP~|gI~|gV] [W_P|W_I|W_V]^T in one pass (the tile kernel of
// gemm_tile.hpp built with SLIME_GEMM_ADD), instead of a bf16 GEMM output and a
// separate sum over the state.
#define SLIME_GEMM_ADD
#include "gemm_tile.hpp"

namespace slime {

hipError_t launch_gemm_add_f32(int dtype, const GemmArgs& a, const float* add, hipStream_t s) {
    if (!gemm_uses_mfma(dtype, a) || a.N != a.ncol || a.act[0] != 0 || !add) return hipErrorInvalidValue;
    int n_cu = 0;
    if (hipError_t e = device_cu_count(&n_cu); e != hipSuccess) return e;
    const int ntiles = (a.M / kBM) * (a.N / kBN);
    const int grid = ntiles < n_cu ? ntiles : n_cu;  // one persistent WG per CU
    if (dtype == 1)
        hipLaunchKernelGGL(gemm_mfma_add_kernel<bf16_t>, dim3(grid), dim3(kThreads), 0, s, a, add);
    else
        hipLaunchKernelGGL(gemm_mfma_add_kernel<float>, dim3(grid), dim3(kThreads), 0, s, a, add);
    return hipGetLastError();
}

}  // namespace slime
