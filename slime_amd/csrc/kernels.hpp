// kernels.hpp — host-side launchers for the gfx950 CA kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slime {

constexpr int kHeads = 8;  // NUM_HEADS, slime/core/pseudopod.cu:15

// Compute units of the current device, queried once per device and cached (the
// persistent kernels size their grids by it).
hipError_t device_cu_count(int* n_cu);

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
// One output plane (N = ncol, identity) written as fp32 out[0] = A Bt^T + add, add of
// out[0]'s layout (in place allowed); MFMA shapes only (else hipErrorInvalidValue).
hipError_t launch_gemm_add_f32(int dtype, const GemmArgs& a, const float* add, hipStream_t s);
// As launch_gemm, and every output plane with the GELU activation is also written
// before it to `pre` (that plane's layout); MFMA shapes only (else hipErrorInvalidValue).
hipError_t launch_gemm_tape(int dtype, const GemmArgs& a, void* pre, hipStream_t s);

// The perception input of the reference's S1 (pvi_chain = 2): S = the toroidal 3x3
// neighbourhood sum of every channel of X, [B][G][G][C] in the storage type
// (multi_head_ca_kernel sums the neighbourhood before the product,
// slime/core/pseudopod.cu:62-91). S must not alias X.
hipError_t launch_neighbourhood_sum(int dtype, const void* X, void* S, int B, int G, int C,
                                    hipStream_t s);

// ---- per-batch scaled, transposed weights -------------------------------------
// Wt[b][p*C + n][k] = cvt( scale_p(b, k) * Wtm[pod(b)][p*C + n][k] ), where the
// mass scale applies only to planes that consume the state (scale[b][k / D]).
struct WeightPrepArgs {
    const float* Wtm;     // [pods][nplanes*C][C] fp32 masters, already transposed
    const float* scale;   // [2][B][H] high then low parts (scale = hi + lo), or nullptr
    void* Wt;             // [B][nplanes*C][C]
    int B, C, D, per_pod, nplanes;
    unsigned scaled_planes;  // bit p set: plane p is multiplied by the scale
};
hipError_t launch_weight_prep(int dtype, const WeightPrepArgs& a, hipStream_t s);

// ---- S2-S6 fused stencil --------------------------------------------------------
struct StencilArgs {
    const void* X;           // [B][G][G][C] state (stored, before scale)
    const float* scale_in;   // [2][B][H] deferred mass scale for X, high then low parts
                             // (scale = hi + lo to ~2^-48); nullptr = 1
    const void* P;
    const void* I;
    const void* V;
    void* Y;                 // [B][G][G][C] unscaled output (storage type, or fp32)
    int y_f32;               // 1: Y is fp32 regardless of the state's storage type
    const float* K;          // [pods][H][9]
    const float* mu;         // [pods][H] or [pods][G][G][H]
    const float* sigma;
    const float* M;          // [pods][H][H]
    // bf16 state, D = 64 only: the potential's 9-tap weights as a band table,
    // [pods][H][3 kernel rows][A_hi, B_hi, A_lo, B_lo] with A = bf16 K[3r] | K[3r+1] << 16
    // and B = K[3r+2] (stencil_kband_bytes / fill_stencil_kband, stencil_band.hpp).
    const void* kband;
    // bf16 state, D = 64 only: 16 counters (tile tickets per XCD, then finished
    // workgroups per XCD), zero before a launch; each launch leaves them zero. Launches
    // that share them must be stream-ordered.
    unsigned* sched;
    double* part_in;         // [B][H][tiles]  sum of scaled X per tile
    double* part_out;        // [B][H][tiles]  sum of stored Y per tile
    int B, G, D, per_pod, per_cell;
    float dt;
    int growth_fn;           // 0 bell, 1 Gaussian, 2 U exp(-U^2) (growth_args, stencil.hip)
    // The backward's tape step only (bf16 state, D = 64, fp32 Y, bell growth): with T set
    // the kernel also sums, per (b, head, tile), Y^2, Y T and T^2 of the stored Y and the
    // target T [B][G][G][C] (storage type), each product exact in fp64, into
    // loss_part [B][H][tiles][3] (the loss then needs no pass of its own over Y and T).
    const void* T;
    double* loss_part;
};
int stencil_tiles_per_batch(int G);
// Host-side table for StencilArgs::kband: bytes for `pods` pods, and its contents
// from K [pods][H][9] (fp32), each weight split into bf16 hi + lo.
size_t stencil_kband_bytes(int pods);
void fill_stencil_kband(const float* K, int pods, uint32_t* out);
hipError_t launch_stencil(int dtype, const StencilArgs& a, hipStream_t s);

// ---- S7 mass conservation ------------------------------------------------------------
// scale[b][h] = |sum_out| > 1e-6 ? sum_in / sum_out : 1, reduced in fixed order,
// written as two floats per (b, h): scale_out[0][b][h] the fp32 rounding of the
// fp64 ratio, scale_out[1][b][h] the fp32 rounding of the rest. A scale applied
// as x * hi + x * lo carries no rounding bias from step to step, so the mass of a
// long chain of steps does not drift with the rounding of the ratio.
// scale64_out (may be nullptr): the same factor as one fp64 value per (b, h).
hipError_t launch_mass_finalize(const double* part_in, const double* part_out, int BH, int tiles,
                                double* mass_in, double* mass_out, float* scale_out,
                                double* scale64_out, hipStream_t s);
hipError_t launch_fill_f64(double* p, int n, double v, hipStream_t s);
// Conservation 1 (per cell and head, slime/core/pseudopod.cu:160-165,196-203), between
// the stencil and launch_mass_finalize: y (the stencil's unscaled output, fp32 when
// y_f32 is set, else the storage type) is renormalised in place per (cell, head) to
// the head sum of x scaled by `scale` ([2][B][H], nullptr = 1), and the per-tile sums
// of part_out ([B][H][tiles], the stencil's layout) are rewritten from the result.
hipError_t launch_cell_conserve(int dtype, const void* x, const float* scale, void* y, int y_f32,
                                double* part_out, int B, int G, int D, hipStream_t s);
// y[i] = cvt((scale[0][b][h] + scale[1][b][h]) * x[i]) over the whole state; x is
// fp32 when x_f32 is set, else in the storage type.
hipError_t launch_rescale(int dtype, const void* x, int x_f32, const float* scale, void* y, int B,
                          int G, int C, int D, hipStream_t s);

// ---- E1-E5 fitness --------------------------------------------------------------------
struct FitnessArgs {
    const void* hist;   // state 0 of the history, each state [B][G][G][C]
    long long t_stride; // bytes from state t to state t + 1 (may be negative)
    int T, B, G, D;
    double* gram_part;  // [B*H][chunks][D*D]
    double* mom_part;   // [B*H][chunks][T][3]: sum x_t, sum x_t^2, sum x_{t-1} x_t
    int chunks;
    float* erank;       // [B][H]
    float* coh;
    float* fitness;
    int* sweeps;        // [B][H] Jacobi sweeps used (may be nullptr)
    // [T][B*H] (may be nullptr): state t of the history is scales[t] times the stored
    // values per (b, h); the moments and the last state's Gram are scaled in fp64.
    const double* scales;
};
int fitness_chunks(int G);
hipError_t launch_fitness(int dtype, const FitnessArgs& a, hipStream_t s);
// Allocation-free fitness (slime_ca_fitness_static): the partial sums live in a
// static device buffer of kFitnessScratchBytes per GPU. fitness_static_chunks: the
// largest chunk count <= fitness_chunks(G) that divides the grid's 64-cell stages
// and whose [B*H][chunks] Gram and moment partials fit in that buffer (0: none
// fits). fitness_static_scratch: the buffer's device address on the current device
// (hipErrorNoBinaryForGpu unless it is a gfx950), looked up on the device's first
// call and cached.
constexpr size_t kFitnessScratchBytes = size_t(32) << 20;
size_t fitness_partial_bytes(int B, int D, int T, int chunks);
int fitness_static_chunks(int B, int G, int D, int T);
hipError_t fitness_static_scratch(void** ptr);
// launch_fitness on the static scratch (f.gram_part and f.mom_part are set here).
// Outside graph capture, a call on another stream than the previous call's waits for
// that call's kernels (a per-device event recorded after each launch), so calls from
// several streams do not overwrite each other's partials; under capture the caller
// orders its replays.
hipError_t launch_fitness_static(int dtype, FitnessArgs f, hipStream_t s);

// ---- backward of one step under the MSE loss (backward.hip) --------------------------------
struct BackwardArgs {
    // forward tape (one step from X, parallel projections, scale 1 on X)
    const void* X;           // [B][G][G][C] input state (storage type)
    const void* P;           // post-activation projections (storage type)
    const void* I;
    const void* V;
    const void* Ipre;        // I before the GELU (storage type)
    const float* Y;          // [B][G][G][C] unscaled step output, fp32
    const void* T;           // target (storage type)
    const float* scale;      // [2][B*H] conservation scale r = hi + lo (high, then low parts)
    const float* K;          // parameters, layouts as StencilArgs
    const float* mu;
    const float* sigma;
    const float* M;
    int B, G, D, per_pod, pods, per_cell;
    float dt;
    float inv_n;             // 1 / (B G^2 C)
    // work buffers
    double* lpart;           // [B*H][lchunks][3]
    int lchunks;             // backward_loss_chunks(G), or the stencil's tiles per batch when
                             // loss_fused
    // loss_fused: lpart holds the tape stencil's per-tile sums of Y^2, Y T, T^2 and
    // ysum_part its per-tile sums of Y ([B*H][lchunks], the mass partials), from which
    // the loss finalize forms the loss sums; no loss-partial pass runs.
    int loss_fused;
    const double* ysum_part;
    float* coef;             // [B*H][3]: gY = (coef0 + coef2) (gY' - coef1), coef0 + coef2 the
                             // scale r (or 1 under the guard); coef1 also enters gX
    double* loss_bh;         // [B*H] sum of squared errors
    float* gU;               // [B][G][G][C] fp32
    float* gVt;              // [B][G][G][C] fp32
    float* att;              // [B][G][G][H][9] attention weights
    float* gS;               // [B][G][G][H][9] score gradients
    void* G3;                // [B][G][G][3C] gradients of P~, I~, V (storage type)
    float* gXd;              // [B][G][G][C] direct part of dL/dX
    float* ppart;            // [pods][H][nW][backward_part_floats()]
    int nW;                  // workgroups per pod in the cell pass
    float* gcell;            // per-cell growth: [B][G][G][H][2]
    // outputs (device, fp32, parameter layouts; may be nullptr)
    float* gK;
    float* gmu;
    float* gsigma;
    float* gM;
};
struct DwArgs {
    float* part;             // [pods * chunks_per_pod][C][3C]
    int C, pods, chunks_per_pod;
    long long rows_per_pod;
    long long rows_per_chunk;  // backward_dw_rows_per_chunk
    float* gWP;              // [pods][C][C] each, may be nullptr
    float* gWI;
    float* gWV;
};
int backward_loss_chunks(int G);
int backward_part_floats();
// Row chunks of the weight-gradient reduction (split over rows, added in order).
long long backward_dw_rows_per_chunk(int dtype, int C, long long rows_per_pod);
int backward_dw_chunks_per_pod(int dtype, int C, long long rows_per_pod);
hipError_t launch_backward_stencil(int dtype, const BackwardArgs& a, hipStream_t s);
hipError_t launch_backward_dw(int dtype, const BackwardArgs& a, const DwArgs& d, hipStream_t s);
hipError_t launch_backward_final(int dtype, const float* gXd, const void* gXp, float* gX, long long n,
                                 hipStream_t s);

// ---- organism adapters (slime/core/organism.cu:691-743) -----------------------------
hipError_t launch_init_from_field(int dtype, const float* conc, void* X, int G, int C,
                                  hipStream_t s);
hipError_t launch_field_from_state(int dtype, const void* X, float* conc, int G, int C,
                                   hipStream_t s);
hipError_t launch_organism_report(const double* mass_out, const float* erank, int H,
                                  float* mass_buffer, float* erank_out, hipStream_t s);

// ---- component pool (slime_pool; slime/memory/pool.cu, slime/core/organism.cu) --------
struct PoolArgs {
    int capacity, genome_size;
    int* id;
    float* fitness;
    float* coherence;
    float* hunger;
    int* age;
    int* alive;
    float* genome;     // [capacity][genome_size]
    float* gradients;  // [capacity][genome_size]
    int* counters;     // active, spawned, culled
};
hipError_t launch_pool_init(const PoolArgs& p, hipStream_t s);
hipError_t launch_pool_set_fitness(const PoolArgs& p, const float* fit, const float* coh, int n, int heads,
                                   int generation, float* fit_hist, float* coh_hist, hipStream_t s);
hipError_t launch_hunger(const float* coh, float* hunger, int n, hipStream_t s);
hipError_t launch_pool_age(const PoolArgs& p, hipStream_t s);
hipError_t launch_pool_cull(const PoolArgs& p, float fitness_threshold, float hunger_threshold, hipStream_t s);
hipError_t launch_pool_spawn(const PoolArgs& p, int parent, float rate, hipStream_t s);
hipError_t launch_pool_spawn_wave(const PoolArgs& p, float probability, int generation, hipStream_t s);

}  // namespace slime
