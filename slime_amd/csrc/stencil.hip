// stencil.hip — stages S2-S6 of the CA step fused into one pass over HBM, plus
// the per-tile partial sums that drive S7 (mass conservation).
//
// Reference math, per batch b, head h, cell (y, x), channel c (toroidal
// neighbours n_k = ((y+dy) mod G, (x+dx) mod G), k = 3(dy+1)+(dx+1)):
//   S2  U   = sum_k K[h][k] X_h(n_k)              slime/core/pseudopod.cu:168-180
//   S3  g   = 2 exp(-((U-mu)/(sigma+1e-7))^2) - 1  failed_attempts/warp_ca.cu:49-56
//   S4  a_k = softmax_k( <P_h(y,x), I_h(n_k)> / sqrt(D) )
//                                                  failed_attempts/pseudopod.cu:208-251
//   S5  Vt  = sum_k a_k V_h(n_k)                  failed_attempts/pseudopod.cu:295-311
//   S6  Z_h = X_h + dt g Vt ;  Y_o = sum_h M[o][h] Z_h
//                                                  slime/core/pseudopod.cu:186-187,231-251
// The toroidal halo tile follows slime/kernels/triton_impl.cu:90-105.
//
// One workgroup owns a 4x8 cell tile of one batch and walks the 8 heads. Per
// head it stages the 6x10 halo of X_h and V_h (fp32, X already multiplied by
// the deferred mass scale), I_h and the centre P_h (storage type, rows padded by
// 16 B) in LDS; computes the 32x9 attention weights; then each thread sweeps a
// run of 4 cells of one tile row for two adjacent channels with a 3x3 register
// window (each halo value is read from LDS 3 times per run, not 9 per cell) and
// accumulates its share of all eight mixed outputs Y_o in registers (64 per
// thread, which keeps the kernel at 2+ waves per SIMD without spills). After the last head the outputs are rounded to
// the storage type, written once, and the tile's per-head sums of the scaled
// input and of the stored output go to global partial buffers (wave64 DPP
// reductions, then a cross-wave pass through LDS).
#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

constexpr int kTileY = 4, kTileX = 8;  // tile (cells)
constexpr int kHaloY = kTileY + 2, kHaloX = kTileX + 2;
constexpr int kHaloCells = kHaloY * kHaloX;
constexpr int kTileCells = kTileY * kTileX;
constexpr int kRun = 4;                // cells per thread along x
constexpr int kAStride = 12;           // floats per cell in the attention buffer

__device__ __forceinline__ int wrapi(int v, int G) { return v < 0 ? v + G : (v >= G ? v - G : v); }

template <typename T, int D>
struct Layout {
    static constexpr int kCE = 16 / (int)sizeof(T);         // elements per 16-byte chunk
    static constexpr int kCPR = D / kCE;                    // chunks per (cell, head) row
    static constexpr int kRowPad = D + kCE;                 // padded row (elements) for I, P
    static constexpr int kThreads = (4 * D) < 64 ? 64 : 4 * D;
    static constexpr int kActive = 4 * D;                   // threads with a (row, pair) task
    static constexpr int kWaves = kThreads / 64;
    static constexpr int offX = 0;
    static constexpr int offV = offX + kHaloCells * D * 4;
    static constexpr int offI = offV + kHaloCells * D * 4;
    static constexpr int offP = offI + kHaloCells * kRowPad * (int)sizeof(T);
    static constexpr int offA = offP + kTileCells * kRowPad * (int)sizeof(T);
    static constexpr int offR = offA + kTileCells * kAStride * 4;
    static constexpr int kBytes = offR + kWaves * 16 * 4;
};

// Dot product of two padded LDS rows of D channels.
template <typename T, int D>
__device__ __forceinline__ float row_dot(const T* a, const T* b) {
    float acc = 0.f;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int c = 0; c < D; c += 8) {
            const uint4 va = *reinterpret_cast<const uint4*>(a + c);
            const uint4 vb = *reinterpret_cast<const uint4*>(b + c);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, va.x),
                                                  __builtin_bit_cast(bf16x2_v, vb.x), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, va.y),
                                                  __builtin_bit_cast(bf16x2_v, vb.y), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, va.z),
                                                  __builtin_bit_cast(bf16x2_v, vb.z), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, va.w),
                                                  __builtin_bit_cast(bf16x2_v, vb.w), acc, false);
        }
    } else {
#pragma unroll
        for (int c = 0; c < D; c += 4) {
            const float4 va = *reinterpret_cast<const float4*>(a + c);
            const float4 vb = *reinterpret_cast<const float4*>(b + c);
            acc = __builtin_fmaf(va.x, vb.x, acc);
            acc = __builtin_fmaf(va.y, vb.y, acc);
            acc = __builtin_fmaf(va.z, vb.z, acc);
            acc = __builtin_fmaf(va.w, vb.w, acc);
        }
    }
    return acc;
}

// Converts one 16-byte chunk to fp32 (times s) and writes it to LDS.
template <typename T>
__device__ __forceinline__ void chunk_to_f32(float* dst, uint4 v, float s) {
    if constexpr (sizeof(T) == 2) {
        float4 lo = make_float4(bf16lo(v.x) * s, bf16hi(v.x) * s, bf16lo(v.y) * s, bf16hi(v.y) * s);
        float4 hi = make_float4(bf16lo(v.z) * s, bf16hi(v.z) * s, bf16lo(v.w) * s, bf16hi(v.w) * s);
        reinterpret_cast<float4*>(dst)[0] = lo;
        reinterpret_cast<float4*>(dst)[1] = hi;
    } else {
        float4 f = __builtin_bit_cast(float4, v);
        f.x *= s;
        f.y *= s;
        f.z *= s;
        f.w *= s;
        *reinterpret_cast<float4*>(dst) = f;
    }
}

// TY: storage type of the unscaled output; fp32 when the caller rescales it into
// the final bf16 state (one rounding instead of two).
template <typename T, int D, typename TY>
__global__ __launch_bounds__((Layout<T, D>::kThreads), 2) void stencil_kernel(StencilArgs a) {
    using L = Layout<T, D>;
    constexpr int H = kHeads;
    constexpr int C = H * D;
    constexpr int kPairs = D / 2;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    float* sX = reinterpret_cast<float*>(lds + L::offX);
    float* sV = reinterpret_cast<float*>(lds + L::offV);
    T* sI = reinterpret_cast<T*>(lds + L::offI);
    T* sP = reinterpret_cast<T*>(lds + L::offP);
    float* sA = reinterpret_cast<float*>(lds + L::offA);
    float* sR = reinterpret_cast<float*>(lds + L::offR);

    const int tid = threadIdx.x;
    const int G = a.G;
    const int tiles_x = G / kTileX;
    const int tpb = (G / kTileY) * tiles_x;
    const int nwg = a.B * tpb;
    int t = blockIdx.x;
    if ((nwg & 7) == 0) t = (t & 7) * (nwg >> 3) + (t >> 3);  // contiguous tile runs per XCD
    const int b = t / tpb;
    const int tile = t % tpb;
    const int ty0 = (tile / tiles_x) * kTileY, tx0 = (tile % tiles_x) * kTileX;
    const int pod = b / a.per_pod;

    const T* Xg = static_cast<const T*>(a.X);
    const T* Pg = static_cast<const T*>(a.P);
    const T* Ig = static_cast<const T*>(a.I);
    const T* Vg = static_cast<const T*>(a.V);
    const long long batch_base = (long long)b * G * G;

    // Phase-B task: a run of 4 cells of one tile row, two adjacent channels.
    const bool active = tid < L::kActive;
    const int cp = tid % kPairs;
    const int grp = tid / kPairs;  // 0..7 when active
    const int ry = grp >> 1;
    const int rx0 = (grp & 1) * kRun;
    const int c0 = 2 * cp;

    float y[H][kRun][2];
#pragma unroll
    for (int o = 0; o < H; ++o)
#pragma unroll
        for (int x = 0; x < kRun; ++x) y[o][x][0] = y[o][x][1] = 0.f;
    float xin[H] = {};

    const float inv_sqrt_d = 1.0f / __builtin_sqrtf((float)D);
    constexpr float kLog2e = 1.4426950408889634f;
    const float sqrt_log2e = __builtin_sqrtf(kLog2e);

    for (int h = 0; h < H; ++h) {
        const float s_in = a.scale_in ? a.scale_in[b * H + h] : 1.0f;
        // ---- phase 0: stage the halo tiles of head h --------------------------------
        constexpr int kHaloChunks = kHaloCells * L::kCPR;
        constexpr int kTotal = 3 * kHaloChunks + kTileCells * L::kCPR;
#pragma unroll 2
        for (int q = tid; q < kTotal; q += L::kThreads) {
            int arr, cell, ch, gy, gx;
            if (q < 3 * kHaloChunks) {
                arr = q / kHaloChunks;
                const int r = q - arr * kHaloChunks;
                cell = r / L::kCPR;
                ch = r - cell * L::kCPR;
                gy = wrapi(ty0 + cell / kHaloX - 1, G);
                gx = wrapi(tx0 + cell % kHaloX - 1, G);
            } else {
                arr = 3;
                const int r = q - 3 * kHaloChunks;
                cell = r / L::kCPR;
                ch = r - cell * L::kCPR;
                gy = ty0 + cell / kTileX;
                gx = tx0 + cell % kTileX;
            }
            const long long off = (batch_base + (long long)gy * G + gx) * C + h * D + ch * L::kCE;
            if (arr == 0) {
                const uint4 v = *reinterpret_cast<const uint4*>(Xg + off);
                chunk_to_f32<T>(sX + cell * D + ch * L::kCE, v, s_in);
            } else if (arr == 1) {
                const uint4 v = *reinterpret_cast<const uint4*>(Vg + off);
                chunk_to_f32<T>(sV + cell * D + ch * L::kCE, v, 1.0f);
            } else if (arr == 2) {
                *reinterpret_cast<uint4*>(sI + cell * L::kRowPad + ch * L::kCE) =
                    *reinterpret_cast<const uint4*>(Ig + off);
            } else {
                *reinterpret_cast<uint4*>(sP + cell * L::kRowPad + ch * L::kCE) =
                    *reinterpret_cast<const uint4*>(Pg + off);
            }
        }
        __syncthreads();

        // ---- phase A: attention scores (S4), k-major so lanes walk adjacent cells --
#pragma unroll 1
        for (int i = tid; i < 9 * kTileCells; i += L::kThreads) {
            const int k = i / kTileCells, cell = i % kTileCells;
            const int cy = cell / kTileX, cx = cell % kTileX;
            const int nb = (cy + k / 3) * kHaloX + (cx + k % 3);
            sA[cell * kAStride + k] =
                row_dot<T, D>(sP + cell * L::kRowPad, sI + nb * L::kRowPad) * inv_sqrt_d;
        }
        __syncthreads();
#pragma unroll 1
        for (int cell = tid; cell < kTileCells; cell += L::kThreads) {
            float* s = sA + cell * kAStride;
            float m = s[0];
#pragma unroll
            for (int k = 1; k < 9; ++k) m = fmaxf(m, s[k]);
            float e[9], sum = 0.f;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                e[k] = exp2_fast((s[k] - m) * kLog2e);
                sum += e[k];
            }
            const float inv = 1.0f / sum;
#pragma unroll
            for (int k = 0; k < 9; ++k) s[k] = e[k] * inv;
        }
        __syncthreads();

        // ---- phase B: potential, growth, propagation, update, head mixing --------
        float xacc = 0.f;
        if (active) {
            float kw[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) kw[k] = a.K[(pod * H + h) * 9 + k];
            float mw[H];
#pragma unroll
            for (int o = 0; o < H; ++o) mw[o] = a.M[(pod * H + o) * H + h];
            float ga = 0.f, gb = 0.f;
            if (!a.per_cell) {
                ga = sqrt_log2e / (a.sigma[pod * H + h] + 1e-7f);
                gb = a.mu[pod * H + h] * ga;
            }
            const float dt = a.dt, two_dt = 2.0f * a.dt;

            float2 xw[3][3], vw[3][3];
#pragma unroll
            for (int dy = 0; dy < 3; ++dy)
#pragma unroll
                for (int dx = 0; dx < 2; ++dx) {
                    const int hc = (ry + dy) * kHaloX + rx0 + dx;
                    xw[dy][dx] = *reinterpret_cast<const float2*>(sX + hc * D + c0);
                    vw[dy][dx] = *reinterpret_cast<const float2*>(sV + hc * D + c0);
                }
#pragma unroll
            for (int x = 0; x < kRun; ++x) {
#pragma unroll
                for (int dy = 0; dy < 3; ++dy) {
                    const int hc = (ry + dy) * kHaloX + rx0 + x + 2;
                    xw[dy][2] = *reinterpret_cast<const float2*>(sX + hc * D + c0);
                    vw[dy][2] = *reinterpret_cast<const float2*>(sV + hc * D + c0);
                }
                const float* ap = sA + (ry * kTileX + rx0 + x) * kAStride;
                const float4 a0 = reinterpret_cast<const float4*>(ap)[0];
                const float4 a1 = reinterpret_cast<const float4*>(ap)[1];
                const float a8 = ap[8];
                const float aw[9] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w, a8};
                if (a.per_cell) {
                    const long long pi =
                        (((long long)pod * G + ty0 + ry) * G + tx0 + rx0 + x) * H + h;
                    ga = sqrt_log2e / (a.sigma[pi] + 1e-7f);
                    gb = a.mu[pi] * ga;
                }
                float z[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    float u = 0.f, vt = 0.f;
#pragma unroll
                    for (int k = 0; k < 9; ++k) {
                        const float2 xv = xw[k / 3][k % 3];
                        const float2 vv = vw[k / 3][k % 3];
                        u = __builtin_fmaf(kw[k], e ? xv.y : xv.x, u);
                        vt = __builtin_fmaf(aw[k], e ? vv.y : vv.x, vt);
                    }
                    const float tg = __builtin_fmaf(u, ga, -gb);
                    const float ex = exp2_fast(-tg * tg);
                    const float coef = __builtin_fmaf(ex, two_dt, -dt);  // dt * g
                    const float xc = e ? xw[1][1].y : xw[1][1].x;
                    z[e] = __builtin_fmaf(coef, vt, xc);
                    xacc += xc;
                }
#pragma unroll
                for (int o = 0; o < H; ++o) {
                    y[o][x][0] = __builtin_fmaf(mw[o], z[0], y[o][x][0]);
                    y[o][x][1] = __builtin_fmaf(mw[o], z[1], y[o][x][1]);
                }
#pragma unroll
                for (int dy = 0; dy < 3; ++dy) {
                    xw[dy][0] = xw[dy][1];
                    xw[dy][1] = xw[dy][2];
                    vw[dy][0] = vw[dy][1];
                    vw[dy][1] = vw[dy][2];
                }
                // Keep the scheduler from hoisting later columns' LDS reads over
                // this cell: the 128 output accumulators already need half the
                // register budget of a 2-waves-per-SIMD launch.
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int j = 0; j < H; ++j) xin[j] = (j == h) ? xacc : xin[j];
        __syncthreads();  // LDS is restaged for the next head
    }

    // ---- phase C: store Y (storage type) and the tile's mass partial sums ---------
    TY* Yg = static_cast<TY*>(a.Y);
    float ysum[H];
#pragma unroll
    for (int o = 0; o < H; ++o) ysum[o] = 0.f;
    if (active) {
#pragma unroll
        for (int x = 0; x < kRun; ++x) {
            const long long base = (batch_base + (long long)(ty0 + ry) * G + tx0 + rx0 + x) * C + c0;
#pragma unroll
            for (int o = 0; o < H; ++o) {
                const float r0 = Store<TY>::round(y[o][x][0]);
                const float r1 = Store<TY>::round(y[o][x][1]);
                ysum[o] += r0 + r1;
                Store<TY>::store2(Yg + base + o * D, r0, r1);
            }
        }
    }
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int j = 0; j < H; ++j) {
        const float sx = wave_sum(xin[j]);
        const float sy = wave_sum(ysum[j]);
        if (lane == 0) {
            sR[wave * 16 + j] = sx;
            sR[wave * 16 + H + j] = sy;
        }
    }
    __syncthreads();
    if (tid < 2 * H) {
        float s = 0.f;
        for (int w = 0; w < L::kWaves; ++w) s += sR[w * 16 + tid];
        const int j = tid % H;
        float* dst = tid < H ? a.part_in : a.part_out;
        dst[((long long)b * H + j) * tpb + tile] = s;
    }
}

template <typename T, int D, typename TY>
hipError_t launch_tdy(const StencilArgs& a, hipStream_t s) {
    using L = Layout<T, D>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)stencil_kernel<T, D, TY>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int tiles = (a.G / kTileY) * (a.G / kTileX);
    hipLaunchKernelGGL((stencil_kernel<T, D, TY>), dim3(a.B * tiles), dim3(L::kThreads), L::kBytes,
                       s, a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_td(const StencilArgs& a, hipStream_t s) {
    return a.y_f32 ? launch_tdy<T, D, float>(a, s) : launch_tdy<T, D, T>(a, s);
}

template <typename T>
hipError_t launch_t(const StencilArgs& a, hipStream_t s) {
    switch (a.D) {
        case 8: return launch_td<T, 8>(a, s);
        case 16: return launch_td<T, 16>(a, s);
        case 32: return launch_td<T, 32>(a, s);
        case 64: return launch_td<T, 64>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int stencil_tiles_per_batch(int G) { return (G / kTileY) * (G / kTileX); }

hipError_t launch_stencil(int dtype, const StencilArgs& a, hipStream_t s) {
    return dtype == 1 ? launch_t<bf16_t>(a, s) : launch_t<float>(a, s);
}

}  // namespace slime
