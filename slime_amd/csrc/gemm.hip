// gemm.hip — S1 head projections on the gfx950 matrix cores.
//
// Replaces the per-thread triple loops of multi_head_ca_kernel
// (slime/core/pseudopod.cu:41-131) and the 16x16 WMMA fragments of
// tensor_core_ca_kernel / tiled_matmul_kernel (slime/core/pseudopod.cu:256-299,
// slime/kernels/triton_impl.cu:16-60) with one fused [P|I|V] GEMM:
//   P = ReLU(X W_P), I = GELU_tanh(X W_I), V = X W_V      (N = 3C, K = C)
//
// Tile: 256 cells x 256 outputs per 256-thread workgroup (4 waves, each 128x128
// as 4x4 MFMA 32x32 blocks), one persistent workgroup per CU. K advances in
// 64-byte slabs (32 bf16 / 16 fp32) through a 4-stage LDS ring filled by direct
// global->LDS loads (global_load_lds_dwordx4), so three slabs are in flight while
// one is consumed. Operand fragments are double-buffered in registers: while a
// wave issues the 32 MFMAs of slab k from one buffer, it reads slab k+1's
// fragments into the other and issues the loads of slab k+4, so the matrix cores
// never wait for an LDS round trip; one barrier per slab publishes slab k+1 and
// frees the stage of slab k. Each tile row's 64 slab bytes sit as four 16-byte
// chunks XOR-swizzled by the row (gemm_addr.hpp), which keeps the operand reads
// free of LDS bank conflicts. The first MFMA of
// a tile starts from a zero accumulator instead of clearing 256 registers. The
// weights are the MFMA "A" operand: a lane's accumulators hold 4 consecutive
// output channels of one cell. The bf16 epilogue goes through LDS so that stores
// leave as whole 128-byte row segments. Workgroups walk an XCD-contiguous tile
// range, N fastest, so a cell block and one batch's weights are re-read from that
// XCD's L2.
// The tile kernel and its helpers are in gemm_tile.hpp (also built, with an adding
// fp32 epilogue, by gemm_add.hip); this file holds the fallback, the launchers and
// the weight folding.
#include "gemm_tile.hpp"

namespace slime {
namespace {

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
        int n_cu = 0;
        if (hipError_t e = device_cu_count(&n_cu); e != hipSuccess) return e;
        const int ntiles = (a.M / kBM) * (a.N / kBN);
        const int grid = ntiles < n_cu ? ntiles : n_cu;  // one persistent WG per CU
        hipLaunchKernelGGL(gemm_mfma_kernel<T>, dim3(grid), dim3(kThreads), 0, s, a);
    } else {
        const long long total = (long long)a.M * a.N;
        hipLaunchKernelGGL(gemm_simple_kernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           s, a);
    }
    return hipGetLastError();
}

}  // namespace

bool gemm_uses_mfma(int dtype, const GemmArgs& a) {
    // K must fill whole groups of 4 slabs (4 x 64 bytes: 128 bf16 or 64 fp32).
    const int k_group = dtype == 1 ? 128 : 64;
    return a.M % kBM == 0 && a.N % kBN == 0 && a.ncol % kBN == 0 && a.K % k_group == 0 &&
           a.rows_per_batch % kBM == 0;
}

hipError_t launch_gemm(int dtype, const GemmArgs& a, hipStream_t s) {
    const bool mfma = gemm_uses_mfma(dtype, a);
    return dtype == 1 ? launch_t<bf16_t>(a, s, mfma) : launch_t<float>(a, s, mfma);
}

// ---- weight preparation --------------------------------------------------------------
namespace {
constexpr int kPrepBatches = 8;  // batches per thread

// One thread per 8 consecutive k of one (plane, n) row of one pod's masters (the 8
// share a head: D >= 8) and up to kPrepBatches batches of that pod (grid y): the
// masters are read once per thread, and each batch's scaled copy leaves as one
// 16-byte (bf16) or two 16-byte (fp32) stores.
template <typename T>
__global__ __launch_bounds__(256) void weight_prep_kernel(WeightPrepArgs w) {
    const long long per_b = (long long)w.nplanes * w.C * w.C;
    const long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int pods = w.B / w.per_pod;
    if (q * 8 >= per_b * pods) return;
    const int pod = (int)(q * 8 / per_b);
    const long long r = q * 8 - (long long)pod * per_b;
    const int k = (int)(r % w.C);
    const int p = (int)(r / ((long long)w.C * w.C));
    const float* src = w.Wtm + (long long)pod * per_b + r;
    const float4 v0 = *reinterpret_cast<const float4*>(src);
    const float4 v1 = *reinterpret_cast<const float4*>(src + 4);
    const bool scaled = w.scale && ((w.scaled_planes >> p) & 1u);
    const int heads = w.C / w.D, head = k / w.D;
    const int b0 = blockIdx.y * kPrepBatches;
    const int b1 = min(w.per_pod, b0 + kPrepBatches);
#pragma unroll 4
    for (int bb = b0; bb < b1; ++bb) {
        const int b = pod * w.per_pod + bb;
        // scale = hi + lo, applied as w * hi + w * lo with one rounding (the stencil
        // applies the same factor to its reads of the state)
        const float s = scaled ? w.scale[b * heads + head] : 1.0f;
        const float sl = scaled ? w.scale[(long long)w.B * heads + b * heads + head] : 0.0f;
        float o[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(o[e], s, o[e] * sl);
        if constexpr (sizeof(T) == 2) {
            *reinterpret_cast<uint4*>(static_cast<T*>(w.Wt) + (long long)b * per_b + r) =
                make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]),
                           pack_bf16x2(o[6], o[7]));
        } else {
            float* dst = static_cast<float*>(w.Wt) + (long long)b * per_b + r;
            *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
    }
}
}  // namespace

// ---- the reference's perception input: the 3x3 neighbourhood sum -------------------
namespace {
// S[b][y][x][c] = sum over the 9 toroidal neighbours (y+dy, x+dx) of X[b][..][..][c],
// taps in the order k = 3(dy+1)+(dx+1), fp32 sums rounded once to the storage type.
// One thread per 8 consecutive channels of a cell: a wave reads whole 1 KiB (bf16)
// or 2 KiB (fp32) cell rows of each neighbour, and the 8 neighbours shared with the
// adjacent cells come from L2.
template <typename T>
__global__ __launch_bounds__(256) void neighbourhood_sum_kernel(const T* X, T* S, int B, int G, int C) {
    const int groups = C / 8;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)B * G * G * groups) return;
    const long long cell = idx / groups;
    const int c0 = (int)(idx - cell * groups) * 8;
    const long long b = cell / ((long long)G * G);
    const int yx = (int)(cell - b * G * G);
    const int y = yx / G, x = yx - y * G;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int dy = -1; dy <= 1; ++dy) {
        const int yy = y + dy < 0 ? G - 1 : (y + dy == G ? 0 : y + dy);
        for (int dx = -1; dx <= 1; ++dx) {
            const int xx = x + dx < 0 ? G - 1 : (x + dx == G ? 0 : x + dx);
            const T* p = X + ((b * G + yy) * G + xx) * C + c0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float2 v = Store<T>::load2(p + 2 * j);
                acc[2 * j] += v.x;
                acc[2 * j + 1] += v.y;
            }
        }
    }
    T* o = S + cell * C + c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) Store<T>::store2(o + 2 * j, acc[2 * j], acc[2 * j + 1]);
}
}  // namespace

hipError_t launch_neighbourhood_sum(int dtype, const void* X, void* S, int B, int G, int C,
                                    hipStream_t s) {
    const long long total = (long long)B * G * G * (C / 8);
    const dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == 1)
        hipLaunchKernelGGL(neighbourhood_sum_kernel<bf16_t>, grid, dim3(256), 0, s,
                           static_cast<const bf16_t*>(X), static_cast<bf16_t*>(S), B, G, C);
    else
        hipLaunchKernelGGL(neighbourhood_sum_kernel<float>, grid, dim3(256), 0, s,
                           static_cast<const float*>(X), static_cast<float*>(S), B, G, C);
    return hipGetLastError();
}

hipError_t launch_weight_prep(int dtype, const WeightPrepArgs& a, hipStream_t s) {
    const long long units = (long long)(a.B / a.per_pod) * a.nplanes * a.C * a.C / 8;
    const dim3 grid((unsigned)((units + 255) / 256), (unsigned)((a.per_pod + kPrepBatches - 1) / kPrepBatches));
    if (dtype == 1)
        hipLaunchKernelGGL(weight_prep_kernel<bf16_t>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(weight_prep_kernel<float>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace slime
