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

template <int kAct>
__device__ __forceinline__ float act_of(float v) {
    if constexpr (kAct == 1) return v > 0.f ? v : 0.f;
    else if constexpr (kAct == 2) return gelu_tanh(v);
    else return v;
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

// Stores a wave's 128x128 accumulator block: lane (r32, half) holds, for each
// 32x32 block (i, j) and group q, 4 consecutive channels of one cell.
template <typename T, int kAct>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[4][4], T* obase, int ncol) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        T* orow = obase + (long long)j * 32 * ncol;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                store4<T>(orow + i * 32 + 8 * q, act_of<kAct>(acc[i][j][4 * q + 0]),
                          act_of<kAct>(acc[i][j][4 * q + 1]), act_of<kAct>(acc[i][j][4 * q + 2]),
                          act_of<kAct>(acc[i][j][4 * q + 3]));
    }
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

// Issues the direct global->LDS loads (global_load_lds_dwordx4, no VGPR staging)
// of one K slab of a tile into one LDS stage. A wave instruction fills 1 KiB of
// LDS = 8 swizzled tile rows: lane i lands at row R + i/8, physical chunk i%8, so
// it fetches logical chunk (i%8) ^ (i/8) of that row. Wave w issues rows
// (4j + w)*8 .. +8 for j = 0..7 of the cell (A) tile and of the weight (Bt) tile.
template <typename T>
__device__ __forceinline__ void issue_slab(const GemmArgs& g, int tile, int nN, int kslab, int wave,
                                           int lane, unsigned char* stage_base) {
    constexpr int kE = 16 / (int)sizeof(T);            // elements per 16-byte chunk
    constexpr int kSlab = kRowBytes / (int)sizeof(T);  // K elements per slab
    const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
    const long long K = g.K;
    const char* a = reinterpret_cast<const char*>(static_cast<const T*>(g.A) + m0 * K + kslab * kSlab);
    const char* b = reinterpret_cast<const char*>(
        static_cast<const T*>(g.Bt) + (long long)(m0 / g.rows_per_batch) * g.bt_batch_stride + n0 * K +
        kslab * kSlab);
    const int sub = lane >> 3;                         // row within the 8-row group
    const int chunk = (lane & 7) ^ sub;                // logical chunk this lane fetches
    const unsigned lane_off = (unsigned)((sub * K + chunk * kE) * (long long)sizeof(T));
    const unsigned row_bytes = (unsigned)(K * sizeof(T));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int R = (4 * j + wave) * 8;
        __builtin_amdgcn_global_load_lds((gbl_void_t*)(a + R * row_bytes + lane_off),
                                         (lds_void_t*)(stage_base + R * kRowBytes), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int R = (4 * j + wave) * 8;
        __builtin_amdgcn_global_load_lds((gbl_void_t*)(b + R * row_bytes + lane_off),
                                         (lds_void_t*)(stage_base + (kBM + R) * kRowBytes), 16, 0, 0);
    }
}

__device__ __forceinline__ void wait_vmem() {
    // s_waitcnt vmcnt(0): this wave's direct-to-LDS loads have landed.
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

// Persistent: each workgroup walks tiles tile0, tile0 + stride, ... of its XCD's
// contiguous tile range. The first slab of the next tile is fetched during the
// last slab of the current one, so only the epilogue separates two tiles.
template <typename T>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    constexpr int kSlab = kRowBytes / (int)sizeof(T);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int r32 = lane & 31, half = lane >> 5;

    const int nN = g.N / kBN;
    const int ntiles = (g.M / kBM) * nN;
    const int nk = g.K / kSlab;
    // XCD-aware schedule: WG w runs on XCD w % 8 (round-robin dispatch). Each XCD
    // owns a contiguous range of tiles (N fastest), so the N tiles of a cell block
    // and one batch's weights are re-read from that XCD's L2.
    int tile, stride, tile_end;
    if ((gridDim.x & 7) == 0) {
        const int per_xcd_wg = gridDim.x >> 3;
        const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
        const int span = (ntiles + 7) >> 3;
        const int begin = xcd * span;
        tile_end = min(ntiles, begin + span);
        tile = begin + j;
        stride = per_xcd_wg;
    } else {
        tile = blockIdx.x;
        stride = gridDim.x;
        tile_end = ntiles;
    }
    if (tile >= tile_end) return;

    issue_slab<T>(g, tile, nN, 0, wave, lane, lds);
    wait_vmem();
    __syncthreads();
    int stage = 0;

    f32x16 acc[4][4];
    while (true) {
        const int next = tile + stride < tile_end ? tile + stride : -1;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

        for (int kt = 0; kt < nk; ++kt) {
            // All MFMA operands of this slab go to registers before the next slab's
            // direct-to-LDS loads are issued: the compiler orders LDS reads after
            // any outstanding LDS-DMA, so reading first keeps the prefetch in flight
            // during the MFMAs instead of draining it at the first ds_read.
            const unsigned char* base = lds + stage * kStageBytes;
            uint4 wf[4][4], xf[4][4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int chunk = 2 * kk + half;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    wf[kk][i] = *reinterpret_cast<const uint4*>(base + swz(kBM + wn * 128 + i * 32 + r32, chunk));
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xf[kk][j] = *reinterpret_cast<const uint4*>(base + swz(wm * 128 + j * 32 + r32, chunk));
            }
            unsigned char* nxt = lds + (stage ^ 1) * kStageBytes;
            if (kt + 1 < nk)
                issue_slab<T>(g, tile, nN, kt + 1, wave, lane, nxt);
            else if (next >= 0)
                issue_slab<T>(g, next, nN, 0, wave, lane, nxt);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if constexpr (sizeof(T) == 2) {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8_v, wf[kk][i]),
                                __builtin_bit_cast(bf16x8_v, xf[kk][j]), acc[i][j], 0, 0, 0);
                        } else {
                            const f32x4 wv = __builtin_bit_cast(f32x4, wf[kk][i]);
                            const f32x4 xv = __builtin_bit_cast(f32x4, xf[kk][j]);
#pragma unroll
                            for (int s = 0; s < 4; ++s)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[s], xv[s],
                                                                                 acc[i][j], 0, 0, 0);
                        }
                    }
            wait_vmem();
            __syncthreads();
            stage ^= 1;
        }

        // Epilogue: the whole 256-wide N tile lies in one output plane, so the
        // activation is uniform over the tile.
        const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
        const int plane = n0 / g.ncol;
        T* out = static_cast<T*>(g.out[plane]);
        const int col0 = n0 - plane * g.ncol + wn * 128;
        T* obase = out + (long long)(m0 + wm * 128 + r32) * g.ncol + col0 + 4 * half;
        switch (g.act[plane]) {
            case 1: store_tile<T, 1>(acc, obase, g.ncol); break;
            case 2: store_tile<T, 2>(acc, obase, g.ncol); break;
            default: store_tile<T, 0>(acc, obase, g.ncol); break;
        }
        if (next < 0) break;
        tile = next;
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
        static int n_cu = 0;
        if (!n_cu) {
            int dev = 0;
            hipError_t e = hipGetDevice(&dev);
            if (e == hipSuccess) e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
            if (e != hipSuccess) return e;
        }
        const int ntiles = (a.M / kBM) * (a.N / kBN);
        const int grid = ntiles < n_cu ? ntiles : n_cu;  // one persistent WG per CU
        hipLaunchKernelGGL(gemm_mfma_kernel<T>, dim3(grid), dim3(kThreads), 2 * kStageBytes, s, a);
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
    // Four consecutive k per thread: coalesced fp32 reads, 8/16-byte writes.
    const long long per_b = (long long)w.nplanes * w.C * w.C;
    const long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q * 4 >= per_b * w.B) return;
    const long long idx = q * 4;
    const int b = (int)(idx / per_b);
    const long long r = idx - (long long)b * per_b;
    const int k = (int)(r % w.C);
    const int p = (int)(r / ((long long)w.C * w.C));
    const int pod = b / w.per_pod;
    float4 v = *reinterpret_cast<const float4*>(w.Wtm + (long long)pod * per_b + r);
    if (w.scale && ((w.scaled_planes >> p) & 1u)) {
        const float s = w.scale[b * (w.C / w.D) + k / w.D];  // 4 k share one head (D >= 8)
        v.x *= s;
        v.y *= s;
        v.z *= s;
        v.w *= s;
    }
    if constexpr (sizeof(T) == 2)
        reinterpret_cast<uint2*>(w.Wt)[q] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    else
        reinterpret_cast<float4*>(w.Wt)[q] = v;
}
}  // namespace

hipError_t launch_weight_prep(int dtype, const WeightPrepArgs& a, hipStream_t s) {
    const long long quads = (long long)a.B * a.nplanes * a.C * a.C / 4;
    const dim3 grid((unsigned)((quads + 255) / 256));
    if (dtype == 1)
        hipLaunchKernelGGL(weight_prep_kernel<bf16_t>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(weight_prep_kernel<float>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace slime
