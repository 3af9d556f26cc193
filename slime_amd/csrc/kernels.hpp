// kernels.hpp — host-side launchers for the gfx950 CA kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slime {

constexpr int kHeads = 8;  // NUM_HEADS, slime/core/pseudopod.cu:15

// ---- S1 projections ----------------------------------------------------------
// out_p[m][col] = act_p( sum_k A[m][k] * Bt[batch(m)][n][k] ), n = p*ncol + col.
struct GemmArgs {
    const void* A;             // [M][K] rows (cells), K contiguous
    const void* Bt;            // per batch [N][K], K contiguous
    long long bt_batch_stride; // elements between consecutive batches' Bt
    int rows_per_batch;        // rows of A that share one Bt (G*G)
    int M, N, K;
    void* out[3];              // output planes [M][ncol]
    int ncol;                  // columns per plane
    int act[3];                // 0 identity, 1 ReLU, 2 tanh-GELU
};
// Returns true when the MFMA tile kernel handles this shape (else the generic
// kernel runs). dtype: 0 fp32, 1 bf16.
bool gemm_uses_mfma(int dtype, const GemmArgs& a);
hipError_t launch_gemm(int dtype, const GemmArgs& a, hipStream_t s);

// ---- per-batch scaled, transposed weights -------------------------------------
// Wt[b][p*C + n][k] = cvt( scale_p(b, k) * Wtm[pod(b)][p*C + n][k] ), where the
// mass scale applies only to planes that consume the state (scale[b][k / D]).
struct WeightPrepArgs {
    const float* Wtm;     // [pods][nplanes*C][C] fp32 masters, already transposed
    const float* scale;   // [B][H] or nullptr
    void* Wt;             // [B][nplanes*C][C]
    int B, C, D, per_pod, nplanes;
    unsigned scaled_planes;  // bit p set: plane p is multiplied by the scale
};
hipError_t launch_weight_prep(int dtype, const WeightPrepArgs& a, hipStream_t s);

// ---- S2-S6 fused stencil --------------------------------------------------------
struct StencilArgs {
    const void* X;           // [B][G][G][C] state (stored, before scale)
    const float* scale_in;   // [B][H] deferred mass scale for X (nullptr = 1)
    const void* P;
    const void* I;
    const void* V;
    void* Y;                 // [B][G][G][C] unscaled output (storage type, or fp32)
    int y_f32;               // 1: Y is fp32 regardless of the state's storage type
    const float* K;          // [pods][H][9]
    const float* mu;         // [pods][H] or [pods][G][G][H]
    const float* sigma;
    const float* M;          // [pods][H][H]
    // bf16 state, D = 64 only: the potential's 9-tap weights as dense bf16 hi/lo
    // matrices over a 4x8 tile's 6x10 halo, [pods][H][2][32 cells][64 halo rows]
    // (stencil_kmat_bytes / fill_stencil_kmat).
    const void* kmat;
    float* part_in;          // [B][H][tiles]  sum of scaled X per tile
    float* part_out;         // [B][H][tiles]  sum of stored Y per tile
    int B, G, D, per_pod, per_cell;
    float dt;
};
int stencil_tiles_per_batch(int G);
// Host-side table for StencilArgs::kmat: bytes for `pods` pods, and its contents
// from K [pods][H][9] (fp32).
size_t stencil_kmat_bytes(int pods);
void fill_stencil_kmat(const float* K, int pods, uint16_t* out);
hipError_t launch_stencil(int dtype, const StencilArgs& a, hipStream_t s);

// ---- S7 mass conservation ------------------------------------------------------------
// scale[b][h] = |sum_out| > 1e-6 ? sum_in / sum_out : 1, reduced in fixed order.
hipError_t launch_mass_finalize(const float* part_in, const float* part_out, int BH, int tiles,
                                double* mass_in, double* mass_out, float* scale_out,
                                hipStream_t s);
// y[i] = cvt(scale[b][h] * x[i]) over the whole state; x is fp32 when x_f32 is
// set, else in the storage type.
hipError_t launch_rescale(int dtype, const void* x, int x_f32, const float* scale, void* y, int B,
                          int G, int C, int D, hipStream_t s);

// ---- E1-E5 fitness --------------------------------------------------------------------
struct FitnessArgs {
    const void* hist;   // state 0 of the history, each state [B][G][G][C]
    long long t_stride; // bytes from state t to state t + 1 (may be negative)
    int T, B, G, D;
    double* gram_part;  // [B*H][chunks][D*D]
    double* mom_part;   // [B*H][chunks][(T-1)*5]
    int chunks;
    float* erank;       // [B][H]
    float* coh;
    float* fitness;
    int* sweeps;        // [B][H] Jacobi sweeps used (may be nullptr)
};
int fitness_chunks(int G);
hipError_t launch_fitness(int dtype, const FitnessArgs& a, hipStream_t s);

// ---- organism adapters (slime/core/organism.cu:691-743) -----------------------------
hipError_t launch_init_from_field(int dtype, const float* conc, void* X, int G, int C,
                                  hipStream_t s);
hipError_t launch_field_from_state(int dtype, const void* X, float* conc, int G, int C,
                                   hipStream_t s);
hipError_t launch_organism_report(const double* mass_out, const float* erank, int H,
                                  float* mass_buffer, float* erank_out, hipStream_t s);

}  // namespace slime
