// gemm.hip — S1 head projections on the gfx950 matrix cores.
//
// Replaces the per-thread triple loops of multi_head_ca_kernel
// (slime/core/pseudopod.cu:41-131) and the 16x16 WMMA fragments of
// tensor_core_ca_kernel / tiled_matmul_kernel (slime/core/pseudopod.cu:256-299,
// slime/kernels/triton_impl.cu:16-60) with one fused [P|I|V] GEMM:
//   P = ReLU(X W_P), I = GELU_tanh(X W_I), V = X W_V      (N = 3C, K = C)
//
// Tile: 256 cells x 256 outputs per 256-thread workgroup (4 waves, each 128x128
// as 4x4 MFMA 32x32 blocks). K advances 128 bytes per stage (64 bf16 or 32
// fp32), staged through double-buffered LDS (2 x 64 KiB) whose 16-byte chunks
// are XOR-swizzled by row so both the stores and the MFMA operand reads are
// bank-conflict free. The weights are the MFMA "A" operand, so each lane's
// accumulators hold 4 consecutive output channels of one cell (8-byte bf16
// stores). Workgroups are renumbered so each XCD walks a contiguous run of
// tiles with the N tiles of a cell block adjacent: the cell block and that
// batch's weights are then re-read from the XCD's own L2, not HBM.
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

constexpr int kBM = 256, kBN = 256, kThreads = 256;
constexpr int kRowBytes = 128;           // bytes of K per tile row per stage
constexpr int kStageBytes = (kBM + kBN) * kRowBytes;

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * kRowBytes + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 1) return v > 0.f ? v : 0.f;
    if (act == 2) return gelu_tanh(v);
    return v;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<float>(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t* p, float a, float b, float c, float d) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
}

template <typename T>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    constexpr int kElemsPerRow = kRowBytes / sizeof(T);  // K per stage

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    // XCD-aware tile order: WG i runs on XCD i % 8; give each XCD a contiguous
    // range of tiles, N fastest.
    const int nN = g.N / kBN;
    const int nwg = (g.M / kBM) * nN;
    int t = blockIdx.x;
    if ((nwg & 7) == 0) t = (t & 7) * (nwg >> 3) + (t >> 3);
    const int m0 = (t / nN) * kBM;
    const int n0 = (t % nN) * kBN;

    const T* A = static_cast<const T*>(g.A);
    const T* Bt = static_cast<const T*>(g.Bt) + (long long)(m0 / g.rows_per_batch) * g.bt_batch_stride;
    const int K = g.K;

    // Per-thread global chunk sources: chunks 0..7 from A rows, 8..15 from Bt rows.
    const int crow = tid >> 3, cchunk = tid & 7;
    const T* srcA = A + (long long)(m0 + crow) * K + cchunk * (16 / sizeof(T));
    const T* srcB = Bt + (long long)(n0 + crow) * K + cchunk * (16 / sizeof(T));
    const long long rowstep = 32LL * K;

    uint4 pre[16];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            pre[j] = *reinterpret_cast<const uint4*>(srcA + j * rowstep + k0);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            pre[8 + j] = *reinterpret_cast<const uint4*>(srcB + j * rowstep + k0);
    };
    auto lstore = [&](int stage) {
        unsigned char* base = lds + stage * kStageBytes;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int row = j * 32 + crow;  // rows 0..255 A, 256..511 Bt
            *reinterpret_cast<uint4*>(base + swz(row, cchunk)) = pre[j];
        }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nk = K / kElemsPerRow;
    gload(0);
    lstore(0);
    __syncthreads();

    const int r32 = lane & 31, half = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) gload((kt + 1) * kElemsPerRow);
        const unsigned char* base = lds + (kt & 1) * kStageBytes;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int chunk = 2 * kk + half;
            uint4 wf[4], xf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = kBM + wn * 128 + i * 32 + r32;
                wf[i] = *reinterpret_cast<const uint4*>(base + swz(row, chunk));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = wm * 128 + j * 32 + r32;
                xf[j] = *reinterpret_cast<const uint4*>(base + swz(row, chunk));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (sizeof(T) == 2) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8_v, wf[i]), __builtin_bit_cast(bf16x8_v, xf[j]),
                            acc[i][j], 0, 0, 0);
                    } else {
                        const f32x4 wv = __builtin_bit_cast(f32x4, wf[i]);
                        const f32x4 xv = __builtin_bit_cast(f32x4, xf[j]);
#pragma unroll
                        for (int s = 0; s < 4; ++s)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[s], xv[s], acc[i][j],
                                                                             0, 0, 0);
                    }
                }
        }
        if (kt + 1 < nk) lstore((kt + 1) & 1);
        __syncthreads();
    }

    // Epilogue: the whole 256-wide N tile lies in one output plane.
    const int plane = n0 / g.ncol;
    const int act = g.act[plane];
    T* out = static_cast<T*>(g.out[plane]);
    const int col0 = n0 - plane * g.ncol + wn * 128;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const long long m = m0 + wm * 128 + j * 32 + r32;
        T* orow = out + m * g.ncol;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = col0 + i * 32 + 8 * q + 4 * half;
                store4<T>(orow + n, apply_act(acc[i][j][4 * q + 0], act),
                          apply_act(acc[i][j][4 * q + 1], act), apply_act(acc[i][j][4 * q + 2], act),
                          apply_act(acc[i][j][4 * q + 3], act));
            }
    }
}

// Any-shape fallback: one thread per output, fp32 accumulation.
template <typename T>
__global__ __launch_bounds__(256) void gemm_simple_kernel(GemmArgs g) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)g.M * g.N) return;
    const int m = (int)(idx / g.N), n = (int)(idx % g.N);
    const T* a = static_cast<const T*>(g.A) + (long long)m * g.K;
    const T* b = static_cast<const T*>(g.Bt) + (long long)(m / g.rows_per_batch) * g.bt_batch_stride +
                 (long long)n * g.K;
    float acc = 0.f;
    for (int k = 0; k < g.K; ++k) acc = __builtin_fmaf(Store<T>::to_f32(a[k]), Store<T>::to_f32(b[k]), acc);
    const int plane = n / g.ncol, col = n % g.ncol;
    static_cast<T*>(g.out[plane])[(long long)m * g.ncol + col] =
        Store<T>::from_f32(apply_act(acc, g.act[plane]));
}

template <typename T>
hipError_t launch_t(const GemmArgs& a, hipStream_t s, bool mfma) {
    if (mfma) {
        static bool attr_set = false;
        if (!attr_set) {
            hipError_t e = hipFuncSetAttribute((const void*)gemm_mfma_kernel<T>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               2 * kStageBytes);
            if (e != hipSuccess) return e;
            attr_set = true;
        }
        const int nwg = (a.M / kBM) * (a.N / kBN);
        hipLaunchKernelGGL(gemm_mfma_kernel<T>, dim3(nwg), dim3(kThreads), 2 * kStageBytes, s, a);
    } else {
        const long long total = (long long)a.M * a.N;
        hipLaunchKernelGGL(gemm_simple_kernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           s, a);
    }
    return hipGetLastError();
}

}  // namespace

bool gemm_uses_mfma(int dtype, const GemmArgs& a) {
    const int elems_per_stage = dtype == 1 ? 64 : 32;
    return a.M % kBM == 0 && a.N % kBN == 0 && a.ncol % kBN == 0 && a.K % elems_per_stage == 0 &&
           a.rows_per_batch % kBM == 0;
}

hipError_t launch_gemm(int dtype, const GemmArgs& a, hipStream_t s) {
    const bool mfma = gemm_uses_mfma(dtype, a);
    return dtype == 1 ? launch_t<bf16_t>(a, s, mfma) : launch_t<float>(a, s, mfma);
}

// ---- weight preparation --------------------------------------------------------------
namespace {
template <typename T>
__global__ __launch_bounds__(256) void weight_prep_kernel(WeightPrepArgs w) {
    // One thread per output element of Wt[b][p*C + n][k]; k fastest for the store.
    const long long per_b = (long long)w.nplanes * w.C * w.C;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= per_b * w.B) return;
    const int b = (int)(idx / per_b);
    const long long r = idx % per_b;
    const int k = (int)(r % w.C);
    const int pn = (int)(r / w.C);  // p*C + n
    const int p = pn / w.C, n = pn % w.C;
    const int pod = b / w.per_pod;
    float v = w.W[(((long long)pod * w.nplanes + p) * w.C + k) * w.C + n];
    if (w.scale && ((w.scaled_planes >> p) & 1u)) v *= w.scale[b * (w.C / w.D) + k / w.D];
    static_cast<T*>(w.Wt)[idx] = Store<T>::from_f32(v);
}
}  // namespace

hipError_t launch_weight_prep(int dtype, const WeightPrepArgs& a, hipStream_t s) {
    const long long total = (long long)a.B * a.nplanes * a.C * a.C;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == 1)
        hipLaunchKernelGGL(weight_prep_kernel<bf16_t>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(weight_prep_kernel<float>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace slime
