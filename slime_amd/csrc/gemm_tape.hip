// gemm_tape.hip — the forward projections of the backward's tape: P = ReLU(X W_P),
// I = GELU_tanh(X W_I), V = X W_V and the pre-activation I~ = X W_I in one pass (the
// tile kernel of gemm_tile.hpp built with SLIME_GEMM_TAPE: the GELU plane's tiles
// leave through the epilogue twice, before and after the activation), instead of
// the projections and a second GEMM over the W_I plane.
#define SLIME_GEMM_TAPE
#include "gemm_tile.hpp"

namespace slime {

hipError_t launch_gemm_tape(int dtype, const GemmArgs& a, void* pre, hipStream_t s) {
    if (!gemm_uses_mfma(dtype, a) || !pre) return hipErrorInvalidValue;
    int n_cu = 0;
    if (hipError_t e = device_cu_count(&n_cu); e != hipSuccess) return e;
    const int ntiles = (a.M / kBM) * (a.N / kBN);
    const int grid = ntiles < n_cu ? ntiles : n_cu;  // one persistent WG per CU
    if (dtype == 1)
        hipLaunchKernelGGL(gemm_mfma_tape_kernel<bf16_t>, dim3(grid), dim3(kThreads), 0, s, a, pre);
    else
        hipLaunchKernelGGL(gemm_mfma_tape_kernel<float>, dim3(grid), dim3(kThreads), 0, s, a, pre);
    return hipGetLastError();
}

}  // namespace slime
