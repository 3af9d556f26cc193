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
// global->LDS loads (global_load_lds_dwordx4), three slabs ahead of the MFMAs, so
// each slab's load latency hides behind three slabs of MFMA work. The four
// stages are separate LDS arrays: the compiler then knows that reading one stage
// does not wait for the loads still landing in the others. 16-byte chunks are
// XOR-swizzled by row pair, so the DMA writes and the operand reads avoid bank
// conflicts. The weights are the MFMA "A" operand: a lane's accumulators hold 4
// consecutive output channels of one cell. The bf16 epilogue goes through LDS
// so that stores leave as whole 128-byte row segments. Workgroups walk an
// XCD-contiguous tile range, N fastest, so a cell block and one batch's weights
// are re-read from that XCD's L2.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {


template <int R0, int N, typename F>
__device__ __forceinline__ void static_for_gemm(F&& f) {
    if constexpr (R0 < N) {
        f(std::integral_constant<int, R0>{});
        static_for_gemm<R0 + 1, N>(f);
    }
}

constexpr int kBM = 256, kBN = 256, kThreads = 256;
constexpr int kSlabB = 64;                    // bytes of K per tile row per slab
constexpr int kStageB = (kBM + kBN) * kSlabB;  // 32 KiB
constexpr int kAhead = 3;                     // slabs in flight ahead of the MFMAs

// Byte offset of 16-byte chunk c (0..3) of tile row r inside a stage.
__device__ __forceinline__ int swz(int row, int chunk) {
    return row * kSlabB + ((chunk ^ ((row >> 1) & 3)) << 4);
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

// fp32 epilogue: direct 16-byte stores of 4 consecutive channels per lane.
template <int kAct>
__device__ __forceinline__ void store_tile_f32(const f32x16 (&acc)[4][4], float* obase, int ncol) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float* orow = obase + (long long)j * 32 * ncol;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4*>(orow + i * 32 + 8 * q) =
                    make_float4(act_of<kAct>(acc[i][j][4 * q + 0]), act_of<kAct>(acc[i][j][4 * q + 1]),
                                act_of<kAct>(acc[i][j][4 * q + 2]), act_of<kAct>(acc[i][j][4 * q + 3]));
    }
}
constexpr int kStoresF32 = 64;  // global stores per wave per tile (fp32 epilogue)

// bf16 epilogue through LDS: for each 32-row block j and each half of the
// wave's 128 columns, the wave writes its accumulators (MFMA layout, 8-byte
// pieces) into a private LDS region and reads them back row-contiguous, so one
// store instruction writes eight whole 128-byte row segments. Rows are padded
// to 144 bytes: the 8-byte writes of 16 consecutive rows hit distinct banks.
constexpr int kEpiRowB = 144;
constexpr int kEpiWaveB = 32 * kEpiRowB;
constexpr int kStoresBf16 = 32;  // global stores per wave per tile (bf16 epilogue)

template <int kAct>
__device__ __forceinline__ void store_tile_bf16(const f32x16 (&acc)[4][4], bf16_t* obase, int ncol,
                                                unsigned char* ep, int lane) {
    const int r32 = lane & 31, half = lane >> 5;
    unsigned char* wp = ep + r32 * kEpiRowB + half * 8;
    const unsigned char* rp = ep + (lane >> 3) * kEpiRowB + (lane & 7) * 16;
    const unsigned gl = (unsigned)(((lane >> 3) * ncol + (lane & 7) * 8) * 2);
    char* ob = reinterpret_cast<char*>(obase);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = 2 * p + ii;
                    const uint2 v = make_uint2(
                        pack_bf16x2(act_of<kAct>(acc[i][j][4 * q + 0]), act_of<kAct>(acc[i][j][4 * q + 1])),
                        pack_bf16x2(act_of<kAct>(acc[i][j][4 * q + 2]), act_of<kAct>(acc[i][j][4 * q + 3])));
                    *reinterpret_cast<uint2*>(wp + (ii * 32 + 8 * q) * 2) = v;
                }
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const uint4 v = *reinterpret_cast<const uint4*>(rp + s4 * 8 * kEpiRowB);
                const long long uoff = ((long long)(j * 32 + s4 * 8) * ncol + p * 64) * 2;  // uniform
                *reinterpret_cast<uint4*>(ob + uoff + gl) = v;
            }
        }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// One direct global->LDS load (global_load_lds_dwordx4): 16 bytes per lane from
// gaddr land at LDS byte address lds_base + 16 * lane. Issued through inline asm:
// the compiler would otherwise make every later LDS read wait for all such loads
// still in flight (it cannot tell which stage they fill). The pipeline waits for
// each slab itself (wait_vm) before the barrier that publishes it.
__device__ __forceinline__ void dma16(const void* gaddr, unsigned lds_base) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off"
        :
        : "s"(lds_base), "v"(gaddr)
        : "memory", "m0");
}

__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const lds_void_t*)p;
}

// Issues the direct global->LDS loads of slab ks of a tile into one stage. A wave
// instruction fills 1 KiB of LDS = 16 tile rows of 64 bytes: lane l lands at row
// R + l/4, physical chunk l%4, so it fetches logical chunk (l%4) ^ ((l/8)%4) of
// that row. Wave w issues row groups (4j + w)*16, j = 0..7: A rows, then Bt rows.
template <typename T>
__device__ __forceinline__ void issue_slab(const GemmArgs& g, int tile, int nN, int ks, int wave,
                                           int lane, unsigned char* stage) {
    constexpr int kE = 16 / (int)sizeof(T);
    constexpr int kSlabE = kSlabB / (int)sizeof(T);
    const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
    const long long K = g.K;
    const char* a = reinterpret_cast<const char*>(static_cast<const T*>(g.A) + m0 * K + ks * kSlabE);
    const char* b = reinterpret_cast<const char*>(
        static_cast<const T*>(g.Bt) + (long long)(m0 / g.rows_per_batch) * g.bt_batch_stride + n0 * K +
        ks * kSlabE);
    const int sub = lane >> 2;
    const int chunk = (lane & 3) ^ ((lane >> 3) & 3);
    const unsigned lane_off = (unsigned)((sub * K + chunk * kE) * (long long)sizeof(T));
    const unsigned row_bytes = (unsigned)(K * sizeof(T));
    const unsigned sbase = lds_addr(stage);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int R = (4 * j + wave) * 16;
        dma16(a + R * row_bytes + lane_off, sbase + R * kSlabB);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int R = (4 * j + wave) * 16;
        dma16(b + R * row_bytes + lane_off, sbase + (kBM + R) * kSlabB);
    }
}
constexpr int kDmaPerSlab = 8;  // DMA instructions per wave per slab

// s_waitcnt vmcnt(n) for the counts the pipeline needs (immediate operand).
__device__ __forceinline__ void wait_vm(int n) {
    // simm16: vmcnt[3:0] | expcnt(7)[6:4] | lgkmcnt(15)[11:8] | vmcnt[5:4] at [15:14]
#define SLIME_VMCNT(n) ((((n) & 15) | ((((n) >> 4) & 3) << 14)) | 0x0F70)
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(0)); break;
        case 8: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(8)); break;
        case 16: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(16)); break;
        case 32: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(32)); break;
        case 40: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(40)); break;
        case 48: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(48)); break;
        default: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(0)); break;
    }
#undef SLIME_VMCNT
}

// Persistent: each workgroup walks tiles tile0, tile0 + stride, ... of its XCD's
// contiguous range. Slab s of every tile lives in stage s % 4; slabs of the next
// tile are fetched while the current tile finishes, so tiles follow each other
// with only the epilogue in between.
// Workgroup barrier for LDS data only: __syncthreads() would also wait for every
// outstanding vector-memory operation (its release fence covers the direct loads
// of later slabs and the previous tile's stores), draining the pipeline.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // s_waitcnt lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <typename T>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) unsigned char st0[kStageB];
    __shared__ __attribute__((aligned(16))) unsigned char st1[kStageB];
    __shared__ __attribute__((aligned(16))) unsigned char st2[kStageB];
    __shared__ __attribute__((aligned(16))) unsigned char st3[kStageB];
    constexpr int kSlabE = kSlabB / (int)sizeof(T);
    constexpr bool kBf16 = sizeof(T) == 2;
    constexpr int kStores = kBf16 ? kStoresBf16 : kStoresF32;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS addresses
    const int wm = wave & 1, wn = wave >> 1;
    const int r32 = lane & 31, half = lane >> 5;

    const int nN = g.N / kBN;
    const int ntiles = (g.M / kBM) * nN;
    const int nk = g.K / kSlabE;  // slabs per tile, a multiple of 4
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

    auto stage_ptr = [&](int s) -> unsigned char* {
        return s == 0 ? st0 : s == 1 ? st1 : s == 2 ? st2 : st3;
    };
    // Prologue: the first kAhead slabs of the first tile.
    for (int s = 0; s < kAhead; ++s) issue_slab<T>(g, tile, nN, s, wave, lane, stage_ptr(s));
    bool stores_pending = false;  // the previous tile's epilogue stores follow slabs 0..2

    f32x16 acc[4][4];
    while (true) {
        const int next = tile + stride < tile_end ? tile + stride : -1;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

        for (int kb = 0; kb < nk; kb += 4) {
            static_for_gemm<0, 4>([&](auto sc) {
                constexpr int S = decltype(sc)::value;
                unsigned char* cur = S == 0 ? st0 : S == 1 ? st1 : S == 2 ? st2 : st3;
                unsigned char* fill = S == 0 ? st3 : S == 1 ? st0 : S == 2 ? st1 : st2;  // (S+3)%4
                const int kt = kb + S;
                // This wave's loads of slab kt have landed once only the younger
                // ones remain outstanding: slabs kt+1, kt+2 (when they exist) and,
                // for the first three slabs after an epilogue, its stores.
                const bool has1 = kt + 1 < nk || next >= 0;
                const bool has2 = kt + 2 < nk || next >= 0;
                int younger = (has1 ? kDmaPerSlab : 0) + (has2 ? kDmaPerSlab : 0);
                if (stores_pending && kt < kAhead) younger = kStores <= 32 ? younger + kStores : 0;
                wait_vm(younger);
                lds_barrier();  // every wave's part of slab kt is in LDS; slab kt-1 is consumed
                // Refill the stage of slab kt-1 with slab kt+3 (this tile or the next).
                if (kt + kAhead < nk)
                    issue_slab<T>(g, tile, nN, kt + kAhead, wave, lane, fill);
                else if (next >= 0)
                    issue_slab<T>(g, next, nN, kt + kAhead - nk, wave, lane, fill);
                if (kt + 1 >= kAhead) stores_pending = false;
                uint4 wf[2][4], xf[2][4];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int chunk = 2 * kk + half;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        wf[kk][i] = *reinterpret_cast<const uint4*>(cur + swz(kBM + wn * 128 + i * 32 + r32, chunk));
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        xf[kk][j] = *reinterpret_cast<const uint4*>(cur + swz(wm * 128 + j * 32 + r32, chunk));
                }
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            if constexpr (kBf16) {
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
            });
        }

        // Epilogue: the whole 256-wide N tile lies in one output plane, so the
        // activation is uniform over the tile.
        const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
        const int plane = n0 / g.ncol;
        T* out = static_cast<T*>(g.out[plane]);
        const int col0 = n0 - plane * g.ncol + wn * 128;
        if constexpr (kBf16) {
            // The last slab's stage (3) is free once every wave has read it; the
            // other three are receiving the next tile's first slabs.
            lds_barrier();
            unsigned char* ep = st3 + wave * kEpiWaveB;
            bf16_t* obase = reinterpret_cast<bf16_t*>(out) + (long long)(m0 + wm * 128) * g.ncol + col0;
            switch (g.act[plane]) {
                case 1: store_tile_bf16<1>(acc, obase, g.ncol, ep, lane); break;
                case 2: store_tile_bf16<2>(acc, obase, g.ncol, ep, lane); break;
                default: store_tile_bf16<0>(acc, obase, g.ncol, ep, lane); break;
            }
        } else {
            float* obase = reinterpret_cast<float*>(out) + (long long)(m0 + wm * 128 + r32) * g.ncol +
                           col0 + 4 * half;
            switch (g.act[plane]) {
                case 1: store_tile_f32<1>(acc, obase, g.ncol); break;
                case 2: store_tile_f32<2>(acc, obase, g.ncol); break;
                default: store_tile_f32<0>(acc, obase, g.ncol); break;
            }
        }
        stores_pending = true;
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
        static int n_cu = 0;
        if (!n_cu) {
            int dev = 0;
            hipError_t e = hipGetDevice(&dev);
            if (e == hipSuccess) e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
            if (e != hipSuccess) return e;
        }
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
