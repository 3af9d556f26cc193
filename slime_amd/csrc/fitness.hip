// fitness.hip — E1-E5: fitness = effective_rank x coherence per (batch, head).
//
// Reference:
//   E1 Gram      A_h = (1/N) sum_cells x_h x_h^T   failed_attempts/pseudopod.cu:366-384
//                (over the last state of the history; per head, not head-averaged)
//   E2 Jacobi    two-sided Jacobi, skip |a_pq| <= 1e-6, <= 30 sweeps, stop when
//                sum |a_pq| < 1e-6 * n              failed_attempts/pseudopod.cu:391-436,
//                                                   slime/kernels/warp_ca.cu:20,51-63
//                sigma_i = sqrt|lambda_i|           slime/kernels/warp_ca.cu:101-103
//   E3 rank      exp(-sum p log(p+1e-7)), p = sigma/(sum sigma + 1e-7)
//                                                   slime/kernels/warp_ca.cu:118-143
//   E4 coherence (mean_t Pearson(X_t, X_{t-1}) + 1) / 2, t = 1..T-1
//                                                   slime/core/organism.cu:256-257
//   E5 fitness   erank * coh                        slime/kernels/warp_ca.cu:219
//
// The reference launches SVD, rank and coherence as dynamic-parallelism children
// of one parent (slime/kernels/warp_ca.cu:178-226). Here two stream-ordered
// kernels do the work: a wide pass over the history that writes per-chunk fp64
// Gram and moment partials, then one wave per (batch, head) that reduces them in
// fixed order, runs the cyclic Jacobi on the fp64 matrix in LDS, and finishes
// rank, coherence and fitness.
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

constexpr int kCellsPerStage = 64;

// State t of the history starts t * f.t_stride bytes after f.hist. The stride may be
// negative: two separately allocated states form a history of two.
template <typename T>
__device__ __forceinline__ const T* history_state(const FitnessArgs& f, int t) {
    return reinterpret_cast<const T*>(static_cast<const char*>(f.hist) + t * f.t_stride);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Per (batch, head, chunk of cells): the D x D Gram partial of the last state and
// the lag-1 moments of every consecutive pair of states. Products of the fp32
// values are exact in fp64 and accumulate in fp64, so the partials carry no
// accumulation error that the Jacobi solve could amplify on a nearly singular Gram
// (small eigenvalues enter the rank through their square roots).
template <typename T, int D>
__global__ __launch_bounds__(256) void fitness_partial_kernel(FitnessArgs f) {
    constexpr int H = kHeads;
    constexpr int C = H * D;
    constexpr int kCE = 16 / (int)sizeof(T);   // elements per 16-byte load
    constexpr int kCPR = D / kCE;               // 16-byte loads per cell of one head
    constexpr int kBS = 4;                      // Gram block edge per thread
    constexpr int kBlk = D / kBS;               // blocks per side (16 at D = 64)
    static_assert(kBlk * kBlk <= 256, "one Gram block per thread");
    __shared__ __attribute__((aligned(16))) float sx[kCellsPerStage * D];
    __shared__ double sred[4][5];

    const int bh = blockIdx.x, chunk = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x;
    const long long cells = (long long)f.G * f.G;
    const long long cpc = cells / f.chunks;
    const long long c_begin = chunk * cpc;
    const T* last = history_state<T>(f, f.T - 1);

    // ---- Gram partial of the last state -----------------------------------------
    const bool gact = tid < kBlk * kBlk;
    const int bi = tid / kBlk, bj = tid % kBlk;
    double g[kBS][kBS];
#pragma unroll
    for (int i = 0; i < kBS; ++i)
#pragma unroll
        for (int j = 0; j < kBS; ++j) g[i][j] = 0.0;
    for (long long c0 = c_begin; c0 < c_begin + cpc; c0 += kCellsPerStage) {
        for (int q = tid; q < kCellsPerStage * kCPR; q += 256) {
            const int cell = q / kCPR, ch = q % kCPR;
            const uint4 v = *reinterpret_cast<const uint4*>(
                last + ((long long)b * cells + c0 + cell) * C + h * D + ch * kCE);
            float* dst = sx + cell * D + ch * kCE;
            if constexpr (sizeof(T) == 2) {
                *reinterpret_cast<float4*>(dst) =
                    make_float4(bf16lo(v.x), bf16hi(v.x), bf16lo(v.y), bf16hi(v.y));
                *reinterpret_cast<float4*>(dst + 4) =
                    make_float4(bf16lo(v.z), bf16hi(v.z), bf16lo(v.w), bf16hi(v.w));
            } else {
                *reinterpret_cast<uint4*>(dst) = v;
            }
        }
        __syncthreads();
        if (gact) {
            for (int cell = 0; cell < kCellsPerStage; ++cell) {
                const float4 xi = *reinterpret_cast<const float4*>(sx + cell * D + bi * kBS);
                const float4 xj = *reinterpret_cast<const float4*>(sx + cell * D + bj * kBS);
                const double di[4] = {xi.x, xi.y, xi.z, xi.w};
                const double dj[4] = {xj.x, xj.y, xj.z, xj.w};
#pragma unroll
                for (int i = 0; i < kBS; ++i)
#pragma unroll
                    for (int j = 0; j < kBS; ++j) g[i][j] = __builtin_fma(di[i], dj[j], g[i][j]);
            }
        }
        __syncthreads();
    }
    if (gact) {
        double* gp = f.gram_part + ((long long)bh * f.chunks + chunk) * D * D;
#pragma unroll
        for (int i = 0; i < kBS; ++i)
#pragma unroll
            for (int j = 0; j < kBS; ++j) gp[(bi * kBS + i) * D + bj * kBS + j] = g[i][j];
    }

    // ---- lag-1 moments over the whole history ---------------------------------------
    // Per t = 1..T-1: sum a, sum b, sum ab, sum aa, sum bb with a = x_{t-1}, b = x_t.
    const int npair = f.T - 1;
    double* mp = f.mom_part + ((long long)bh * f.chunks + chunk) * npair * 5;
    const long long nelem = cpc * D;
    const long long base = ((long long)b * cells + c_begin) * C + h * D;
    for (int t = 1; t < f.T; ++t) {
        double sa = 0.0, sb = 0.0, sab = 0.0, saa = 0.0, sbb = 0.0;
        const T* xa = history_state<T>(f, t - 1) + base;
        const T* xb = history_state<T>(f, t) + base;
        for (long long e = tid; e < nelem; e += 256) {
            const long long off = (e / D) * C + (e % D);
            const double va = Store<T>::to_f32(xa[off]);
            const double vb = Store<T>::to_f32(xb[off]);
            sa += va;
            sb += vb;
            sab = __builtin_fma(va, vb, sab);
            saa = __builtin_fma(va, va, saa);
            sbb = __builtin_fma(vb, vb, sbb);
        }
        const double vals[5] = {sa, sb, sab, saa, sbb};
        const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
        for (int m = 0; m < 5; ++m) {
            const double w = wave_sum_f64(vals[m]);
            if (lane == 0) sred[wave][m] = w;
        }
        __syncthreads();
        if (tid < 5) mp[(t - 1) * 5 + tid] = sred[0][tid] + sred[1][tid] + sred[2][tid] + sred[3][tid];
        __syncthreads();
    }
}

// One wave per (batch, head): fixed-order reduction of the partials, the cyclic
// two-sided Jacobi solve in fp64 LDS, then rank, coherence and fitness.
//
// The solve visits the pairs (p, q) in the reference's cyclic row order
// (failed_attempts/pseudopod.cu:391-436) and skips |a_pq| <= 1e-6. That absolute
// threshold makes the converged diagonal depend on the visiting order when the
// Gram is nearly singular, so the order is kept rather than a parallel one. In a
// rotation the entries outside the 2x2 block (p, q) change only in rows p, q and
// columns p, q, each read and written by one lane (lane i owns A[i][p], A[i][q],
// A[p][i], A[q][i]), and the block itself takes its exact diagonal form; one
// barrier per rotation publishes the new diagonal to the next rotation.
template <int D>
__global__ __launch_bounds__(64) void fitness_finalize_kernel(FitnessArgs f) {
    constexpr int kLd = D + 1;  // padded row
    __shared__ double A[D * kLd];
    __shared__ double sv[D];
    __shared__ double rho[64];

    const int bh = blockIdx.x, lane = threadIdx.x;
    const double ncell = (double)f.G * f.G;
    const double tol = 1e-6;

    // Fixed-order reduction of the Gram partials.
    for (int e = lane; e < D * D; e += 64) {
        double s = 0.0;
        for (int c = 0; c < f.chunks; ++c) s += f.gram_part[((long long)bh * f.chunks + c) * D * D + e];
        A[(e / D) * kLd + e % D] = s / ncell;
    }
    __syncthreads();

    int sweeps = 0;
    for (int sweep = 0; sweep < 30; ++sweep) {
        ++sweeps;
        double off = 0.0;
        for (int p = 0; p < D - 1; ++p)
            for (int q = p + 1; q < D; ++q) {
                const double app = A[p * kLd + p], aqq = A[q * kLd + q], apq = A[p * kLd + q];
                off += fabs(apq);
                if (fabs(apq) > tol) {  // uniform across the wave
                    const double tau = (aqq - app) / (2.0 * apq);
                    const double t = tau >= 0.0 ? 1.0 / (tau + sqrt(1.0 + tau * tau))
                                                : -1.0 / (-tau + sqrt(1.0 + tau * tau));
                    const double c = 1.0 / sqrt(1.0 + t * t), s = t * c;
                    const int i = lane;
                    if (i < D && i != p && i != q) {
                        const double aip = A[i * kLd + p], aiq = A[i * kLd + q];
                        A[i * kLd + p] = c * aip - s * aiq;
                        A[i * kLd + q] = s * aip + c * aiq;
                        const double api = A[p * kLd + i], aqi = A[q * kLd + i];
                        A[p * kLd + i] = c * api - s * aqi;
                        A[q * kLd + i] = s * api + c * aqi;
                    }
                    if (lane == 0) {
                        A[p * kLd + p] = c * c * app + s * s * aqq - 2.0 * c * s * apq;
                        A[q * kLd + q] = s * s * app + c * c * aqq + 2.0 * c * s * apq;
                        A[p * kLd + q] = 0.0;
                        A[q * kLd + p] = 0.0;
                    }
                    __syncthreads();
                }
            }
        if (off < tol * D) break;
    }

    // Coherence from the moment partials.
    const int npair = f.T - 1;
    const double n = ncell * D;
    for (int t = lane; t < npair; t += 64) {
        double m[5] = {0, 0, 0, 0, 0};
        for (int c = 0; c < f.chunks; ++c)
            for (int j = 0; j < 5; ++j)
                m[j] += f.mom_part[(((long long)bh * f.chunks + c) * npair + t) * 5 + j];
        const double cov = m[2] - m[0] * m[1] / n;
        const double va = m[3] - m[0] * m[0] / n;
        const double vb = m[4] - m[1] * m[1] / n;
        const double den = sqrt(fmax(va, 0.0) * fmax(vb, 0.0));
        rho[t] = den > 0.0 ? cov / den : 0.0;
    }
    if (lane < D) sv[lane] = sqrt(fabs(A[lane * kLd + lane]));
    __syncthreads();
    if (lane == 0) {
        for (int i = 1; i < D; ++i) {  // descending insertion sort
            const double v = sv[i];
            int j = i - 1;
            while (j >= 0 && sv[j] < v) {
                sv[j + 1] = sv[j];
                --j;
            }
            sv[j + 1] = v;
        }
        double sum = 0.0;
        for (int i = 0; i < D; ++i) sum += sv[i];
        double ent = 0.0;
        for (int i = 0; i < D; ++i) {
            const double p = sv[i] / (sum + 1e-7);
            ent += -p * log(p + 1e-7);
        }
        const double er = exp(ent);
        double rs_ = 0.0;
        for (int t = 0; t < npair; ++t) rs_ += rho[t];
        const double coh = (rs_ / npair + 1.0) * 0.5;
        f.erank[bh] = (float)er;
        f.coh[bh] = (float)coh;
        f.fitness[bh] = (float)(er * coh);
        if (f.sweeps) f.sweeps[bh] = sweeps;
    }
}

template <typename T, int D>
hipError_t launch_td(const FitnessArgs& f, hipStream_t s) {
    hipLaunchKernelGGL((fitness_partial_kernel<T, D>), dim3(f.B * kHeads, f.chunks), dim3(256), 0, s, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(fitness_finalize_kernel<D>, dim3(f.B * kHeads), dim3(64), 0, s, f);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const FitnessArgs& f, hipStream_t s) {
    switch (f.D) {
        case 8: return launch_td<T, 8>(f, s);
        case 16: return launch_td<T, 16>(f, s);
        case 32: return launch_td<T, 32>(f, s);
        case 64: return launch_td<T, 64>(f, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int fitness_chunks(int G) {
    const long long stages = (long long)G * G / kCellsPerStage;
    int c = 16;
    while (c > 1 && (stages % c) != 0) --c;
    return stages >= 1 ? c : 0;
}

hipError_t launch_fitness(int dtype, const FitnessArgs& f, hipStream_t s) {
    return dtype == 1 ? launch_t<bf16_t>(f, s) : launch_t<float>(f, s);
}

}  // namespace slime
