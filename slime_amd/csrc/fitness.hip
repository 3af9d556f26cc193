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
// kernels do the work: a wide pass over the history that writes per-chunk Gram
// and moment partials, then one workgroup per (batch, head) that reduces them in
// fixed order, runs a round-robin parallel Jacobi (D/2 disjoint rotations per
// round, D-1 rounds per sweep) on the fp64 matrix in LDS, and finishes rank,
// coherence and fitness.
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

constexpr int kCellsPerStage = 64;

template <typename T, int D>
__global__ __launch_bounds__(256) void fitness_partial_kernel(FitnessArgs f) {
    constexpr int H = kHeads;
    constexpr int C = H * D;
    constexpr int kCE = 16 / (int)sizeof(T);
    constexpr int kCPR = D / kCE;
    constexpr int kBlk = D / 16 > 0 ? D / 16 : 1;   // Gram block grid side (4x4 blocks)
    constexpr int kBS = D / kBlk;                     // block edge (4 when D >= 16)
    __shared__ __attribute__((aligned(16))) float sx[kCellsPerStage * D];
    __shared__ float sred[4][64];

    const int bh = blockIdx.x, chunk = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x;
    const long long cells = (long long)f.G * f.G;
    const long long cpc = cells / f.chunks;
    const long long c_begin = chunk * cpc;
    const long long state = (long long)f.B * cells * C;
    const T* hist = static_cast<const T*>(f.hist);
    const T* last = hist + (long long)(f.T - 1) * state;

    // ---- Gram partial of the last state -----------------------------------------
    const bool gact = tid < kBlk * kBlk;
    const int bi = tid / kBlk, bj = tid % kBlk;
    float g[kBS][kBS];
#pragma unroll
    for (int i = 0; i < kBS; ++i)
#pragma unroll
        for (int j = 0; j < kBS; ++j) g[i][j] = 0.f;
    for (long long c0 = c_begin; c0 < c_begin + cpc; c0 += kCellsPerStage) {
        for (int q = tid; q < kCellsPerStage * kCPR; q += 256) {
            const int cell = q / kCPR, ch = q % kCPR;
            const uint4 v = *reinterpret_cast<const uint4*>(
                last + ((long long)b * cells + c0 + cell) * C + h * D + ch * kCE);
            float* dst = sx + cell * D + ch * kCE;
            if constexpr (sizeof(T) == 2) {
                dst[0] = bf16lo(v.x); dst[1] = bf16hi(v.x); dst[2] = bf16lo(v.y); dst[3] = bf16hi(v.y);
                dst[4] = bf16lo(v.z); dst[5] = bf16hi(v.z); dst[6] = bf16lo(v.w); dst[7] = bf16hi(v.w);
            } else {
                *reinterpret_cast<uint4*>(dst) = v;
            }
        }
        __syncthreads();
        if (gact) {
            for (int cell = 0; cell < kCellsPerStage; ++cell) {
                float xi[kBS], xj[kBS];
#pragma unroll
                for (int i = 0; i < kBS; ++i) {
                    xi[i] = sx[cell * D + bi * kBS + i];
                    xj[i] = sx[cell * D + bj * kBS + i];
                }
#pragma unroll
                for (int i = 0; i < kBS; ++i)
#pragma unroll
                    for (int j = 0; j < kBS; ++j) g[i][j] = __builtin_fmaf(xi[i], xj[j], g[i][j]);
            }
        }
        __syncthreads();
    }
    if (gact) {
        float* gp = f.gram_part + ((long long)bh * f.chunks + chunk) * D * D;
#pragma unroll
        for (int i = 0; i < kBS; ++i)
#pragma unroll
            for (int j = 0; j < kBS; ++j) gp[(bi * kBS + i) * D + bj * kBS + j] = g[i][j];
    }

    // ---- lag-1 moments over the whole history ---------------------------------------
    // Per t = 1..T-1: sum a, sum b, sum ab, sum aa, sum bb with a = x_{t-1}, b = x_t.
    const int npair = f.T - 1;
    float* mp = f.mom_part + ((long long)bh * f.chunks + chunk) * npair * 5;
    const long long nelem = cpc * D;
    for (int t = 1; t < f.T; ++t) {
        float sa = 0.f, sb = 0.f, sab = 0.f, saa = 0.f, sbb = 0.f;
        const T* xa = hist + (long long)(t - 1) * state + ((long long)b * cells + c_begin) * C + h * D;
        const T* xb = xa + state;
        for (long long e = tid; e < nelem; e += 256) {
            const long long off = (e / D) * C + (e % D);
            const float va = Store<T>::to_f32(xa[off]);
            const float vb = Store<T>::to_f32(xb[off]);
            sa += va;
            sb += vb;
            sab = __builtin_fmaf(va, vb, sab);
            saa = __builtin_fmaf(va, va, saa);
            sbb = __builtin_fmaf(vb, vb, sbb);
        }
        const float vals[5] = {sa, sb, sab, saa, sbb};
        const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
        for (int m = 0; m < 5; ++m) {
            const float w = wave_sum(vals[m]);
            if (lane == 0) sred[wave][m] = w;
        }
        __syncthreads();
        if (tid < 5) mp[(t - 1) * 5 + tid] = sred[0][tid] + sred[1][tid] + sred[2][tid] + sred[3][tid];
        __syncthreads();
    }
}

// Round-robin schedule: round r pairs player n-1 with r and (r+k) with (r-k),
// indices mod n-1; every unordered pair meets exactly once in n-1 rounds.
__device__ __forceinline__ void rr_pair(int n, int r, int k, int* p, int* q) {
    int a, b;
    if (k == 0) {
        a = n - 1;
        b = r;
    } else {
        a = (r + k) % (n - 1);
        b = (r - k + (n - 1)) % (n - 1);
    }
    *p = a < b ? a : b;
    *q = a < b ? b : a;
}

template <int D>
__global__ __launch_bounds__(256) void fitness_finalize_kernel(FitnessArgs f) {
    constexpr int kPairs = D / 2;
    constexpr int kLd = D + 1;  // padded row
    __shared__ double A[D * kLd];
    __shared__ double rc[kPairs], rs[kPairs], rapp[kPairs], raqq[kPairs], rapq[kPairs];
    __shared__ int rp[kPairs], rq[kPairs], ract[kPairs];
    __shared__ double offs[kPairs];
    __shared__ double sv[D];
    __shared__ double rho[64];
    __shared__ int done;

    const int bh = blockIdx.x, tid = threadIdx.x;
    const double inv_n = 1.0 / ((double)f.G * f.G);
    const double tol = 1e-6;

    // Fixed-order reduction of the Gram partials.
    for (int e = tid; e < D * D; e += 256) {
        double s = 0.0;
        for (int c = 0; c < f.chunks; ++c) s += (double)f.gram_part[((long long)bh * f.chunks + c) * D * D + e];
        A[(e / D) * kLd + e % D] = s * inv_n;
    }
    if (tid < kPairs) offs[tid] = 0.0;
    if (tid == 0) done = 0;
    __syncthreads();

    int sweeps = 0;
    for (int sweep = 0; sweep < 30; ++sweep) {
        ++sweeps;
        for (int r = 0; r < D - 1; ++r) {
            if (tid < kPairs) {
                int p, q;
                rr_pair(D, r, tid, &p, &q);
                const double app = A[p * kLd + p], aqq = A[q * kLd + q], apq = A[p * kLd + q];
                int act = 0;
                double c = 1.0, s = 0.0;
                if (fabs(apq) > tol) {
                    const double tau = (aqq - app) / (2.0 * apq);
                    const double t = tau >= 0.0 ? 1.0 / (tau + sqrt(1.0 + tau * tau))
                                                : -1.0 / (-tau + sqrt(1.0 + tau * tau));
                    c = 1.0 / sqrt(1.0 + t * t);
                    s = t * c;
                    act = 1;
                }
                offs[tid] += fabs(apq);
                rp[tid] = p;
                rq[tid] = q;
                rc[tid] = c;
                rs[tid] = s;
                ract[tid] = act;
                rapp[tid] = app;
                raqq[tid] = aqq;
                rapq[tid] = apq;
            }
            __syncthreads();
            // Column rotations: A <- A J for every active pair.
            for (int w = tid; w < D * kPairs; w += 256) {
                const int k = w % kPairs, i = w / kPairs;
                if (!ract[k]) continue;
                const int p = rp[k], q = rq[k];
                const double c = rc[k], s = rs[k];
                const double aip = A[i * kLd + p], aiq = A[i * kLd + q];
                A[i * kLd + p] = c * aip - s * aiq;
                A[i * kLd + q] = s * aip + c * aiq;
            }
            __syncthreads();
            // Row rotations: A <- J^T A; the 2x2 block gets its exact diagonal form.
            for (int w = tid; w < D * kPairs; w += 256) {
                const int k = w / D, j = w % D;
                if (!ract[k]) continue;
                const int p = rp[k], q = rq[k];
                const double c = rc[k], s = rs[k];
                if (j == p) {
                    const double app = rapp[k], aqq = raqq[k], apq = rapq[k];
                    A[p * kLd + p] = c * c * app + s * s * aqq - 2.0 * c * s * apq;
                    A[q * kLd + p] = 0.0;
                } else if (j == q) {
                    const double app = rapp[k], aqq = raqq[k], apq = rapq[k];
                    A[q * kLd + q] = s * s * app + c * c * aqq + 2.0 * c * s * apq;
                    A[p * kLd + q] = 0.0;
                } else {
                    const double apj = A[p * kLd + j], aqj = A[q * kLd + j];
                    A[p * kLd + j] = c * apj - s * aqj;
                    A[q * kLd + j] = s * apj + c * aqj;
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            double off = 0.0;
            for (int k = 0; k < kPairs; ++k) off += offs[k];
            done = off < tol * D;
        }
        __syncthreads();
        if (tid < kPairs) offs[tid] = 0.0;
        const int stop = done;
        __syncthreads();
        if (stop) break;
    }

    // Coherence from the moment partials.
    const int npair = f.T - 1;
    const double n = (double)f.G * f.G * D;
    for (int t = tid; t < npair; t += 256) {
        double m[5] = {0, 0, 0, 0, 0};
        for (int c = 0; c < f.chunks; ++c)
            for (int j = 0; j < 5; ++j)
                m[j] += (double)f.mom_part[(((long long)bh * f.chunks + c) * npair + t) * 5 + j];
        const double cov = m[2] - m[0] * m[1] / n;
        const double va = m[3] - m[0] * m[0] / n;
        const double vb = m[4] - m[1] * m[1] / n;
        const double den = sqrt(fmax(va, 0.0) * fmax(vb, 0.0));
        rho[t] = den > 0.0 ? cov / den : 0.0;
    }
    if (tid < D) sv[tid] = sqrt(fabs(A[tid * kLd + tid]));
    __syncthreads();
    if (tid == 0) {
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
    hipLaunchKernelGGL(fitness_finalize_kernel<D>, dim3(f.B * kHeads), dim3(256), 0, s, f);
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
