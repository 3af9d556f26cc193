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
#include <cstring>
#include <mutex>

#include "common.hpp"
#include "fp64.hpp"
#include "kernels.hpp"

// Scratch of the allocation-free entry point slime_ca_fitness_static: the Gram and
// moment partials of one call. One copy per GPU, created when the code object loads
// on that device and held until the process ends; every call on a GPU shares it.
// Calls on different streams are ordered by launch_fitness_static (each waits for the
// previous call's event); calls under graph capture are not, and replays that overlap
// on one GPU race. Host code never takes the array's name as an address (on the host
// it is only a stand-in for the symbol): the device address is looked up once per
// device and kernels receive that pointer.
static __device__ __align__(256) unsigned char scratch[slime::kFitnessScratchBytes];

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

// Up to kTB states are read per pass over a chunk; their sums stay in registers.
constexpr int kTB = 8;

// The 16-byte pieces of state t that thread `tid` owns in the stage whose head-h
// slice starts `stage_off` bytes into each state: piece j is (cell, channel group)
// = divmod(tid + 256 j, D / elements-per-piece). The uniform part of the address
// is one scalar base per state; the per-thread part is a small byte offset that
// does not change between stages or states. Pieces past the stage hold zeros.
template <typename T, int D, int kPPT>
__device__ __forceinline__ void load_pieces(const FitnessArgs& f, int t, long long stage_off, int tid,
                                            uint4 (&x)[kPPT]) {
    constexpr int kCE = 16 / (int)sizeof(T);
    constexpr int kCPR = D / kCE;
    constexpr int kPieces = kCellsPerStage * kCPR;
    constexpr int C = kHeads * D;
    const char* base = static_cast<const char*>(f.hist) + t * f.t_stride + stage_off;
#pragma unroll
    for (int j = 0; j < kPPT; ++j) {
        const int q = tid + 256 * j;
        if (kPieces % 256 == 0 || q < kPieces) {
            const unsigned off = (unsigned)(((q / kCPR) * C + (q % kCPR) * kCE) * (int)sizeof(T));
            x[j] = *reinterpret_cast<const uint4*>(base + off);
        } else {
            x[j] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
}

template <typename T>
__device__ __forceinline__ void unpack_piece(const uint4& v, float (&e)[16 / sizeof(T)]) {
    if constexpr (sizeof(T) == 2) {
        e[0] = bf16lo(v.x), e[1] = bf16hi(v.x), e[2] = bf16lo(v.y), e[3] = bf16hi(v.y);
        e[4] = bf16lo(v.z), e[5] = bf16hi(v.z), e[6] = bf16lo(v.w), e[7] = bf16hi(v.w);
    } else {
        e[0] = __builtin_bit_cast(float, v.x), e[1] = __builtin_bit_cast(float, v.y);
        e[2] = __builtin_bit_cast(float, v.z), e[3] = __builtin_bit_cast(float, v.w);
    }
}

// Per (batch, head, chunk of cells): the D x D Gram partial of the last state, and
// for every state t the sums S1 = sum x_t, S2 = sum x_t^2 and P = sum x_{t-1} x_t
// (P of state 0 is 0), which give the lag-1 moments of each consecutive pair.
// Products of the fp32 values are exact in fp64 and accumulate in fp64, so the
// partials carry no accumulation error that the Jacobi solve could amplify on a
// nearly singular Gram (small eigenvalues enter the rank through their square
// roots). Each pass over the chunk reads states tb - 1 .. tb + kTB - 1 once, with
// 16-byte loads, all of a stage's loads in flight together; the last pass stages
// the last state through LDS for the Gram.
template <typename T, int D>
__global__ __launch_bounds__(256) void fitness_partial_kernel(FitnessArgs f) {
    constexpr int H = kHeads;
    constexpr int kCE = 16 / (int)sizeof(T);   // elements per 16-byte piece
    constexpr int kCPR = D / kCE;               // pieces per cell of one head
    constexpr int kPieces = kCellsPerStage * kCPR;
    constexpr int kPPT = (kPieces + 255) / 256;  // pieces per thread
    constexpr int kBS = 4;                      // Gram block edge per thread
    constexpr int kBlk = D / kBS;               // blocks per side (16 at D = 64)
    static_assert(kBlk * kBlk <= 256, "one Gram block per thread");
    __shared__ __attribute__((aligned(16))) float sx[kCellsPerStage * D];
    __shared__ double sred[4][3 * kTB];

    const int bh = blockIdx.x, chunk = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long long cells = (long long)f.G * f.G;
    const long long cpc = cells / f.chunks;
    const long long c_begin = chunk * cpc;

    const bool gact = tid < kBlk * kBlk;
    const int bi = tid / kBlk, bj = tid % kBlk;
    double g[kBS][kBS];
#pragma unroll
    for (int i = 0; i < kBS; ++i)
#pragma unroll
        for (int j = 0; j < kBS; ++j) g[i][j] = 0.0;

    double* mp = f.mom_part + ((long long)bh * f.chunks + chunk) * f.T * 3;
    for (int tb = 0; tb < f.T; tb += kTB) {
        const int tn = min(kTB, f.T - tb);  // states tb .. tb + tn - 1 in this pass
        const bool last = tb + tn == f.T;
        double s1[kTB], s2[kTB], pr[kTB];
#pragma unroll
        for (int k = 0; k < kTB; ++k) s1[k] = s2[k] = pr[k] = 0.0;
        for (long long c0 = c_begin; c0 < c_begin + cpc; c0 += kCellsPerStage) {
            const long long stage_off = (((long long)b * cells + c0) * (kHeads * D) + h * D) * (long long)sizeof(T);
            uint4 x[kTB + 1][kPPT];  // states tb - 1 .. tb + kTB - 1
            if (tb > 0) {
                load_pieces<T, D, kPPT>(f, tb - 1, stage_off, tid, x[0]);
            } else {
#pragma unroll
                for (int j = 0; j < kPPT; ++j) x[0][j] = make_uint4(0u, 0u, 0u, 0u);
            }
            // Past the last state the loads repeat it (cached); those sums are unused.
#pragma unroll
            for (int k = 0; k < kTB; ++k) load_pieces<T, D, kPPT>(f, min(tb + k, f.T - 1), stage_off, tid, x[k + 1]);
#pragma unroll
            for (int k = 0; k < kTB; ++k)
#pragma unroll
                for (int j = 0; j < kPPT; ++j) {
                    float a[kCE], e[kCE];
                    unpack_piece<T>(x[k][j], a);
                    unpack_piece<T>(x[k + 1][j], e);
#pragma unroll
                    for (int u = 0; u < kCE; ++u) {
                        const double va = a[u], vb = e[u];
                        s1[k] += vb;
                        s2[k] = __builtin_fma(vb, vb, s2[k]);
                        pr[k] = __builtin_fma(va, vb, pr[k]);
                    }
                    // one piece at a time: the converted values stay few
                    __builtin_amdgcn_sched_barrier(0);
                }
            if (last) {
                // x[tn] holds the last state: stage it as fp32 for the Gram.
#pragma unroll
                for (int k = 1; k <= kTB; ++k) {
                    if (k != tn) continue;
#pragma unroll
                    for (int j = 0; j < kPPT; ++j) {
                        const int q = tid + 256 * j;
                        if (kPieces % 256 == 0 || q < kPieces) {
                            float e[kCE];
                            unpack_piece<T>(x[k][j], e);
                            float* dst = sx + (q / kCPR) * D + (q % kCPR) * kCE;
#pragma unroll
                            for (int u = 0; u < kCE; u += 4)
                                *reinterpret_cast<float4*>(dst + u) = make_float4(e[u], e[u + 1], e[u + 2], e[u + 3]);
                        }
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
        }
        // Block sums of this pass's states, in a fixed order (lanes, then waves).
#pragma unroll
        for (int k = 0; k < kTB; ++k) {
            const double v[3] = {wave_sum_f64(s1[k]), wave_sum_f64(s2[k]), wave_sum_f64(pr[k])};
            if (lane == 0) {
                sred[wave][3 * k] = v[0];
                sred[wave][3 * k + 1] = v[1];
                sred[wave][3 * k + 2] = v[2];
            }
        }
        __syncthreads();
        if (tid < 3 * tn) {
            const double sum = sred[0][tid] + sred[1][tid] + sred[2][tid] + sred[3][tid];
            mp[(long long)tb * 3 + tid] = (tb == 0 && tid == 2) ? 0.0 : sum;
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
}

// Value of v in lane l (l uniform), through two 32-bit lane reads.
__device__ __forceinline__ double lane_f64(double v, int l) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// Keeps the compiler from moving LDS accesses across this point. The block is one
// wave and LDS executes a wave's accesses in issue order, so program order is all
// the ordering that one lane's write and another lane's later read need.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// One wave per (batch, head): fixed-order reduction of the partials, the cyclic
// two-sided Jacobi solve in fp64, then rank, coherence and fitness.
//
// The solve visits the pairs (p, q) in the reference's cyclic row order
// (failed_attempts/pseudopod.cu:391-436) and skips |a_pq| <= 1e-6. That absolute
// threshold makes the converged diagonal depend on the visiting order when the
// Gram is nearly singular, so the order is kept rather than a parallel one, and the
// rotation chain is serial. Its latency is kept to the scalar arithmetic: lane i
// holds column p (A[i][p]) and the diagonal (A[i][i]) in registers, so a_pq and
// a_qq of the next pair are lane reads of registers rather than LDS round trips.
// The matrix stays in LDS (exactly symmetric: each new value is written to both
// (i, p) and (p, i)); column q is read from it once per rotation, in parallel with
// the rotation's scalar chain, and column p once per row p. The chain's divisions
// and square roots use the short correctly rounded forms of fp64.hpp, whose
// preconditions every Gram of fp32 data meets.
//
// Skipped pairs cost no serial step: one ballot over column p finds the next pair
// that rotates, and each lane keeps its own share of the off-diagonal sum, added
// across lanes at the end of the sweep (the reference adds the same |a_pq| values
// one by one in visiting order; the two sums can differ in their last bits, and
// only their comparison with 1e-6 n is used). Since a pair at or below 1e-6 is
// never rotated, that sum usually stays above 1e-6 n and the solve runs to its
// 30-sweep limit, the last sweeps rotating nothing; a sweep that rotates nothing
// ends the solve at once with the same matrix and sweep count.
template <int D>
__global__ __launch_bounds__(64) void fitness_finalize_kernel(FitnessArgs f) {
    constexpr int kLd = D + 1;  // padded row
    __shared__ double A[D * kLd];
    __shared__ double rho[64];

    const int bh = blockIdx.x, lane = threadIdx.x;
    const bool own = D == kWave || lane < D;  // lane owns row/column `lane` of the matrix
    const double ncell = (double)f.G * f.G;
    const double tol = 1e-6;
    const int BH = gridDim.x;
    // Per-state factors of a rolled-out history (1 when the states are stored as they are).
    auto scale_of = [&](int t) { return f.scales ? f.scales[(long long)t * BH + bh] : 1.0; };
    const double s_last = scale_of(f.T - 1);
    const double gram_scale = s_last * s_last / ncell;

    // Fixed-order reduction of the Gram partials: element e sums chunks 0, 1, ... in
    // turn; kE elements per lane at once keep the loads independent.
    {
        constexpr int kE = D * D >= 4 * 64 ? 4 : D * D / 64;  // D * D is a multiple of 64
        static_assert(D * D % (kE * 64) == 0, "whole groups of elements");
        const double* gp = f.gram_part + (long long)bh * f.chunks * D * D;
        for (int e0 = 0; e0 < D * D; e0 += kE * 64) {
            double s[kE];
#pragma unroll
            for (int k = 0; k < kE; ++k) s[k] = 0.0;
#pragma unroll 4
            for (int c = 0; c < f.chunks; ++c)
#pragma unroll
                for (int k = 0; k < kE; ++k) s[k] += gp[(long long)c * D * D + e0 + k * 64 + lane];
#pragma unroll
            for (int k = 0; k < kE; ++k) {
                const int e = e0 + k * 64 + lane;
                A[(e / D) * kLd + e % D] = f.scales ? s[k] * gram_scale : s[k] / ncell;
            }
        }
    }
    __syncthreads();

    double diag = own ? A[lane * kLd + lane] : 0.0;
    int sweeps = 0;
    for (int sweep = 0; sweep < 30; ++sweep) {
        ++sweeps;
        double offl = 0.0;  // lane q: sum over the rows p < q of |a_pq| when (p, q) is visited
        bool rotated = false;
        for (int p = 0; p < D - 1; ++p) {
            lds_order();
            double colp = own ? A[lane * kLd + p] : 0.0;  // A[lane][p] = a_p,lane
            // The read has landed before the rotations start; without this the loop
            // head waits for every LDS access in flight, the previous rotation's
            // writes included, on each rotation.
            asm volatile("" : "+v"(colp));
            double app = lane_f64(diag, p);
            for (int q = p + 1;;) {
                // Pairs (p, q..) with |a_pq| <= tol are skipped without changing anything,
                // so the next rotation is at the lowest lane >= q whose column-p entry
                // exceeds tol; the skipped pairs only add their |a_pq| to the sum.
                const bool ahead = own && lane >= q;
                const unsigned long long m = __ballot(ahead && fabs(colp) > tol);
                const int qn = m ? (int)__builtin_ctzll(m) : D;
                if (ahead && lane <= qn) offl += fabs(colp);  // lane qn: the rotated pair's a_pq
                if (qn >= D) break;
                lds_order();
                const double colq = own ? A[lane * kLd + qn] : 0.0;
                const double apq = lane_f64(colp, qn);
                const double aqq = lane_f64(diag, qn);
                double c, s;
                jacobi_rotation<true>(app, aqq, apq, c, s);
                const double app_new = c * c * app + s * s * aqq - 2.0 * c * s * apq;
                const double aqq_new = s * s * app + c * c * aqq + 2.0 * c * s * apq;
                double np = c * colp - s * colq;
                double nq = s * colp + c * colq;
                if (lane == p) {
                    np = app_new;
                    nq = 0.0;
                } else if (lane == qn) {
                    np = 0.0;
                    nq = aqq_new;
                }
                if (own) {
                    A[lane * kLd + p] = np;
                    A[p * kLd + lane] = np;
                    A[lane * kLd + qn] = nq;
                    A[qn * kLd + lane] = nq;
                }
                diag = lane == p ? app_new : (lane == qn ? aqq_new : diag);
                colp = np;
                app = app_new;
                rotated = true;
                q = qn + 1;
            }
        }
        const double off = wave_sum_f64(offl);
        if (off < tol * D) break;
        // A sweep without a rotation leaves the matrix as it found it, so every later
        // sweep repeats it exactly: the solve ends at the sweep limit.
        if (!rotated) {
            sweeps = 30;
            break;
        }
    }
    lds_order();

    // Coherence from the per-state sums: pair t = (t - 1, t) has sum a = S1(t-1),
    // sum b = S1(t), sum ab = P(t), sum aa = S2(t-1), sum bb = S2(t); chunks in order.
    const int npair = f.T - 1;
    const double n = ncell * D;
    for (int t = lane + 1; t < f.T; t += 64) {
        double m[5] = {0, 0, 0, 0, 0};
        for (int c = 0; c < f.chunks; ++c) {
            const double* q = f.mom_part + ((long long)bh * f.chunks + c) * f.T * 3;
            m[0] += q[(t - 1) * 3];
            m[1] += q[t * 3];
            m[2] += q[t * 3 + 2];
            m[3] += q[(t - 1) * 3 + 1];
            m[4] += q[t * 3 + 1];
        }
        if (f.scales) {
            const double sa = scale_of(t - 1), sb = scale_of(t);
            m[0] *= sa;
            m[1] *= sb;
            m[2] *= sa * sb;
            m[3] *= sa * sa;
            m[4] *= sb * sb;
        }
        const double cov = m[2] - m[0] * m[1] / n;
        const double va = m[3] - m[0] * m[0] / n;
        const double vb = m[4] - m[1] * m[1] / n;
        const double den = sqrt(fmax(va, 0.0) * fmax(vb, 0.0));
        rho[t - 1] = den > 0.0 ? cov / den : 0.0;
    }
    double* sv = A;  // the matrix is no longer needed: its first row holds the singular values
    __syncthreads();
    if (own) sv[lane] = sqrt(fabs(diag));
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

size_t fitness_partial_bytes(int B, int D, int T, int chunks) {
    return (size_t)B * kHeads * chunks * ((size_t)D * D + 3 * (size_t)T) * sizeof(double);
}

int fitness_static_chunks(int B, int G, int D, int T) {
    const long long stages = (long long)G * G / kCellsPerStage;
    for (int c = fitness_chunks(G); c >= 1; --c)
        if (stages % c == 0 && fitness_partial_bytes(B, D, T, c) <= kFitnessScratchBytes) return c;
    return 0;
}

namespace {
// Per device: the scratch's device address, and the event and stream of the last
// call that launched outside graph capture.
struct StaticSlot {
    void* addr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool recorded = false;
};
constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
StaticSlot g_static[kMaxDevices];

hipError_t static_slot(StaticSlot** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    StaticSlot& s = g_static[dev];
    if (!s.addr) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return e;
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return hipErrorNoBinaryForGpu;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        e = hipEventCreateWithFlags(&s.done, hipEventDisableTiming);
        if (e != hipSuccess) return e;
        s.addr = p;
    }
    *out = &s;
    return hipSuccess;
}
}  // namespace

hipError_t fitness_static_scratch(void** ptr) {
    std::lock_guard<std::mutex> lock(g_static_mu);
    StaticSlot* s = nullptr;
    const hipError_t e = static_slot(&s);
    if (e == hipSuccess) *ptr = s->addr;
    return e;
}

hipError_t launch_fitness_static(int dtype, FitnessArgs f, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_static_mu);
    StaticSlot* s = nullptr;
    hipError_t e = static_slot(&s);
    if (e != hipSuccess) return e;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess) return e;
    const bool ordered = cap == hipStreamCaptureStatusNone;
    // The previous call's kernels, if they ran on another stream, finish with the
    // scratch before this call's kernels write it.
    if (ordered && s->recorded && s->last != stream) {
        e = hipStreamWaitEvent(stream, s->done, 0);
        if (e != hipSuccess) return e;
    }
    f.gram_part = static_cast<double*>(s->addr);
    f.mom_part = f.gram_part + (size_t)f.B * kHeads * f.chunks * f.D * f.D;
    e = launch_fitness(dtype, f, stream);
    if (e != hipSuccess || !ordered) return e;
    e = hipEventRecord(s->done, stream);
    if (e == hipSuccess) {
        s->last = stream;
        s->recorded = true;
    }
    return e;
}

}  // namespace slime
