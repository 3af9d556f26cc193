// organism.hip — the adapters around the CA step in the reference organism loop:
//   initialize_ca_from_field_kernel  X[y,x,c] = conc[y,x] * sin(0.1 c)
//                                    slime/core/organism.cu:691-720 (the else-branch
//                                    there is unreachable because NUM_HEADS*HEAD_DIM
//                                    == CHANNELS)
//   update_field_from_ca_kernel      conc[y,x] = mean_c X[y,x,c]
//                                    slime/core/organism.cu:723-743
// One wave per cell for the field update (a wave64 DPP sum over the channels).
// organism_report_kernel writes what neural_ca_update_kernel
// (slime/core/organism.cu:617-688) leaves behind per generation: the per-head mass
// buffer and one effective-rank entry of the history.
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void init_from_field_kernel(const float* conc, T* X, int G, int C) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)G * G * C) return;
    const long long cell = idx / C;
    const int c = (int)(idx - cell * C);
    X[idx] = Store<T>::from_f32(conc[cell] * sinf((float)c * 0.1f));
}

template <typename T>
__global__ __launch_bounds__(256) void field_from_state_kernel(const T* X, float* conc, int G, int C) {
    const long long cell = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const bool valid = cell < (long long)G * G;
    float s = 0.f;
    if (valid)
        for (int c = lane; c < C; c += 64) s += Store<T>::to_f32(X[cell * C + c]);
    s = wave_sum(s);
    if (valid && lane == 0) conc[cell] = s / (float)C;
}

// After one organism generation: mass_buffer[h] = conserved mass of head h (may be
// null) and *erank_out = mean over heads of the effective rank, added in head order.
__global__ __launch_bounds__(64) void organism_report_kernel(const double* mass_out,
                                                             const float* erank, int H,
                                                             float* mass_buffer,
                                                             float* erank_out) {
    const int h = threadIdx.x;
    if (mass_buffer && h < H) mass_buffer[h] = (float)mass_out[h];
    if (h == 0) {
        float s = 0.f;
        for (int i = 0; i < H; ++i) s += erank[i];
        *erank_out = s / (float)H;
    }
}

}  // namespace

hipError_t launch_organism_report(const double* mass_out, const float* erank, int H,
                                  float* mass_buffer, float* erank_out, hipStream_t s) {
    hipLaunchKernelGGL(organism_report_kernel, dim3(1), dim3(64), 0, s, mass_out, erank, H,
                       mass_buffer, erank_out);
    return hipGetLastError();
}

hipError_t launch_init_from_field(int dtype, const float* conc, void* X, int G, int C, hipStream_t s) {
    const long long total = (long long)G * G * C;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == 1)
        hipLaunchKernelGGL(init_from_field_kernel<bf16_t>, grid, dim3(256), 0, s, conc,
                           static_cast<bf16_t*>(X), G, C);
    else
        hipLaunchKernelGGL(init_from_field_kernel<float>, grid, dim3(256), 0, s, conc,
                           static_cast<float*>(X), G, C);
    return hipGetLastError();
}

hipError_t launch_field_from_state(int dtype, const void* X, float* conc, int G, int C, hipStream_t s) {
    const dim3 grid((unsigned)(((long long)G * G + 3) / 4));
    if (dtype == 1)
        hipLaunchKernelGGL(field_from_state_kernel<bf16_t>, grid, dim3(256), 0, s,
                           static_cast<const bf16_t*>(X), conc, G, C);
    else
        hipLaunchKernelGGL(field_from_state_kernel<float>, grid, dim3(256), 0, s,
                           static_cast<const float*>(X), conc, G, C);
    return hipGetLastError();
}

}  // namespace slime
