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
#include "stencil_band.hpp"
#include "stencil_sched.hpp"

#include <cstring>
#include <type_traits>

namespace slime {
namespace {

constexpr int kTileY = 4, kTileX = 8;  // tile (cells)
constexpr int kHaloX = kTileX + 2;     // halo rows are 10 cells wide, 6 rows tall
constexpr int kHaloCells = (kTileY + 2) * kHaloX;  // 60
constexpr int kHaloPad = 64;           // halo cells reserved per array
constexpr int kTileCells = kTileY * kTileX;        // 32
constexpr int kRun = 4;                // cells per thread along x in phase B
constexpr int kAStride = 12;           // floats per cell in the attention buffer

__device__ __forceinline__ int wrapi(int v, int G) { return v < 0 ? v + G : (v >= G ? v - G : v); }

// Calls f(std::integral_constant<int, R>) for R = R0..N-1: array indices stay
// compile-time constants, so the staging registers never become a stack array.
template <int R0, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (R0 < N) {
        f(std::integral_constant<int, R0>{});
        static_for<R0 + 1, N>(f);
    }
}

template <typename T, int D>
struct Layout {
    static constexpr int kCE = 16 / (int)sizeof(T);          // elements per 16-byte chunk
    static constexpr int kCPR = D / kCE;                     // chunks per (cell, head) row
    static constexpr int kRowB = D * (int)sizeof(T);         // bytes per (cell, head) row
    static constexpr int kSwz = (kCPR < 8 ? kCPR : 8) - 1;   // chunk XOR mask (I and P rows)
    static constexpr int kThreads = (4 * D) < 64 ? 64 : 4 * D;
    static constexpr int kActive = 4 * D;                    // threads with a phase-B task
    static constexpr int kWaves = kThreads / 64;
    static constexpr int kTPC = kThreads / kTileCells;       // phase-A threads per cell
    // Direct global->LDS staging: one wave instruction fills 1 KiB = kCPI rows.
    static constexpr int kCPI = 64 / kCPR;                   // cells per DMA instruction
    static constexpr int kPCells = kCPI > kTileCells ? kCPI : kTileCells;  // P rows (padded)
    static constexpr int kHG = kHaloPad / kCPI;              // instruction groups per halo array
    static constexpr int kPG = kPCells / kCPI;               // instruction groups of the P tile
    static constexpr int kIA = kHG / kWaves;                 // per wave, per halo array
    static constexpr int kPA = kPG / kWaves;                 // per wave, P tile
    static_assert(kHG % kWaves == 0 && kPG % kWaves == 0, "DMA groups must split over waves");
    static constexpr int kBufB = (3 * kHaloPad + kPCells) * kRowB;
    static constexpr int offX = 0, offV = kHaloPad * kRowB, offI = 2 * kHaloPad * kRowB,
                         offP = 3 * kHaloPad * kRowB;
};

// Direct global->LDS loads: dma16_lds, dma16_lds_nt, wait_vm0 (common.hpp); the kernel
// waits for them (wait_vm0) before the barrier that publishes them.

// Workgroup barrier for LDS data only. __syncthreads() also waits for every
// outstanding vector-memory operation (its release fence covers the direct
// loads still landing in the other staging buffer); this waits for this wave's
// LDS operations (lgkmcnt(0)) and then meets the other waves at s_barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // s_waitcnt lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// S3 in one form for the three growth functions. With U the scaled potential,
//   ex = 2^-(U ga - gb)^2,   dt g = ex (c1 + c2 U) + c0:
//   bell      2 exp(-((U - mu)/(sigma + 1e-7))^2) - 1: ga = sqrt(log2 e) / (sigma + 1e-7),
//             gb = mu ga, c = (-dt, 2 dt, 0)        failed_attempts/warp_ca.cu:49-56
//   Gaussian  exp(-(U - mu)^2 / (2 sigma^2)): ga = sqrt(log2 e) / (sqrt(2) sigma),
//             gb = mu ga, c = (0, dt, 0)           failed_attempts/pseudopod.cu:46-48
//   shipped   U exp(-U^2): ga = sqrt(log2 e), gb = 0, c = (0, 0, dt)
//                                                  slime/core/pseudopod.cu:183
// For the bell, ex (c1 + 0 U) + c0 is the value of ex 2dt - dt, bit for bit.
struct Growth {
    float ga, gb, c0, c1, c2;
};
__device__ __forceinline__ Growth growth_args(int fn, float mu, float sigma, float dt) {
    const float kSqrtLog2e = __builtin_sqrtf(1.4426950408889634f);  // sqrt(log2 e)
    Growth g;
    if (fn == 2) {
        g.ga = kSqrtLog2e;
        g.gb = 0.f;
        g.c0 = 0.f, g.c1 = 0.f, g.c2 = dt;
    } else if (fn == 1) {
        g.ga = kSqrtLog2e / (1.4142135623730951f * sigma);
        g.gb = mu * g.ga;
        g.c0 = 0.f, g.c1 = dt, g.c2 = 0.f;
    } else {
        g.ga = kSqrtLog2e / (sigma + 1e-7f);
        g.gb = mu * g.ga;
        g.c0 = -dt, g.c1 = 2.0f * dt, g.c2 = 0.f;
    }
    return g;
}

template <typename T>
__device__ __forceinline__ float2 lds_pair(const unsigned char* p) {
    if constexpr (sizeof(T) == 2) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
        return make_float2(bf16lo(w), bf16hi(w));
    } else {
        return *reinterpret_cast<const float2*>(p);
    }
}

// Partial dot product of one 16-byte chunk of two rows.
template <typename T>
__device__ __forceinline__ float chunk_dot(uint4 a, uint4 b, float acc) {
    if constexpr (sizeof(T) == 2) {
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.x),
                                              __builtin_bit_cast(bf16x2_v, b.x), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.y),
                                              __builtin_bit_cast(bf16x2_v, b.y), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.z),
                                              __builtin_bit_cast(bf16x2_v, b.z), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.w),
                                              __builtin_bit_cast(bf16x2_v, b.w), acc, false);
    } else {
        const float4 fa = __builtin_bit_cast(float4, a), fb = __builtin_bit_cast(float4, b);
        acc = __builtin_fmaf(fa.x, fb.x, acc);
        acc = __builtin_fmaf(fa.y, fb.y, acc);
        acc = __builtin_fmaf(fa.z, fb.z, acc);
        acc = __builtin_fmaf(fa.w, fb.w, acc);
    }
    return acc;
}

// Sum over groups of kN consecutive lanes (kN = 1, 2, 4 or 8), every lane of the
// group receiving the sum (DPP quad_perm and row_half_mirror steps).
template <int kN>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (kN >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (kN >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (kN >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror
    return v;
}

template <int kN>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (kN >= 2) v = fmaxf(v, dpp_f32<0xB1>(v));
    if constexpr (kN >= 4) v = fmaxf(v, dpp_f32<0x4E>(v));
    if constexpr (kN >= 8) v = fmaxf(v, dpp_f32<0x141>(v));
    return v;
}

// TY: storage type of the unscaled output; fp32 when the caller rescales it into
// the final bf16 state (one rounding instead of two).
template <typename T, int D, typename TY>
__global__ __launch_bounds__((Layout<T, D>::kThreads), 2) void stencil_kernel(StencilArgs a) {
    using L = Layout<T, D>;
    constexpr int H = kHeads;
    constexpr int C = H * D;
    constexpr int kPairs = D / 2;
    // Two staging buffers as separate LDS objects: the compiler can then tell that
    // reading one does not depend on the direct loads landing in the other.
    __shared__ __attribute__((aligned(16))) unsigned char bufA[L::kBufB];
    __shared__ __attribute__((aligned(16))) unsigned char bufB[L::kBufB];
    __shared__ __attribute__((aligned(16))) float sAtt[2][kTileCells * kAStride];
    __shared__ __attribute__((aligned(16))) float sMS[H * kTileCells * 2];
    __shared__ double sR[L::kWaves * 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS addresses
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
    const long long bbase = (long long)b * G * G * C;  // element offset of batch b

    // ---- direct global->LDS staging of one head --------------------------------------
    // Lane l of a DMA instruction covering cells g*kCPI .. +kCPI lands at row
    // g*kCPI + l/kCPR, physical chunk l%kCPR. X and V rows are stored linearly; I
    // and P rows are XOR-swizzled by cell (the score phase reads whole rows of
    // neighbouring cells), so those lanes fetch logical chunk (l%kCPR) ^ (cell&kSwz).
    // Wave w issues groups g = w + k*kWaves. Per-lane element offsets, head 0:
    int hoff_lin[L::kIA], hoff_swz[L::kIA], poff[L::kPA];
    {
        const int ch = lane % L::kCPR;
#pragma unroll
        for (int k = 0; k < L::kIA; ++k) {
            const int cell = (wave + k * L::kWaves) * L::kCPI + lane / L::kCPR;
            const int gc = cell < kHaloCells ? cell : kHaloCells - 1;  // padding rows
            const int gy = wrapi(ty0 + gc / kHaloX - 1, G), gx = wrapi(tx0 + gc % kHaloX - 1, G);
            const int base = (gy * G + gx) * C;
            hoff_lin[k] = base + ch * L::kCE;
            hoff_swz[k] = base + (ch ^ (cell & L::kSwz)) * L::kCE;
        }
#pragma unroll
        for (int k = 0; k < L::kPA; ++k) {
            const int cell = (wave + k * L::kWaves) * L::kCPI + lane / L::kCPR;
            const int gc = cell < kTileCells ? cell : kTileCells - 1;  // padding rows
            poff[k] = ((ty0 + gc / kTileX) * G + tx0 + gc % kTileX) * C +
                      (ch ^ (cell & L::kSwz)) * L::kCE;
        }
    }
    const char* srcX = reinterpret_cast<const char*>(static_cast<const T*>(a.X) + bbase);
    const char* srcV = reinterpret_cast<const char*>(static_cast<const T*>(a.V) + bbase);
    const char* srcI = reinterpret_cast<const char*>(static_cast<const T*>(a.I) + bbase);
    const char* srcP = reinterpret_cast<const char*>(static_cast<const T*>(a.P) + bbase);
    // Byte offsets (within the batch entry) of this lane's 16-byte pieces.
    unsigned boff_lin[L::kIA], boff_swz[L::kIA], boff_p[L::kPA];
#pragma unroll
    for (int k = 0; k < L::kIA; ++k) {
        boff_lin[k] = (unsigned)hoff_lin[k] * (unsigned)sizeof(T);
        boff_swz[k] = (unsigned)hoff_swz[k] * (unsigned)sizeof(T);
    }
#pragma unroll
    for (int k = 0; k < L::kPA; ++k) boff_p[k] = (unsigned)poff[k] * (unsigned)sizeof(T);
    auto issue_head = [&](int h, unsigned char* buf) {
        const unsigned hb = (unsigned)(h * D * (int)sizeof(T));
#pragma unroll
        for (int k = 0; k < L::kIA; ++k) {
            const unsigned row = lds_addr(buf) + (wave + k * L::kWaves) * 1024;
            dma16_lds(srcX, boff_lin[k] + hb, row + L::offX);
            dma16_lds(srcV, boff_lin[k] + hb, row + L::offV);
            dma16_lds(srcI, boff_swz[k] + hb, row + L::offI);
        }
#pragma unroll
        for (int k = 0; k < L::kPA; ++k)
            dma16_lds(srcP, boff_p[k] + hb, lds_addr(buf) + L::offP + (wave + k * L::kWaves) * 1024);
    };

    // Per-head parameters (and per-cell growth parameters) go to LDS once, before
    // any direct load is issued: reading them later from global memory would make
    // the in-order vector-memory counter wait for the next head's staging.
    __shared__ float sK[H * 9], sMW[H * H], sGa[H], sGb[H], sScale[H], sScaleLo[H];
    {
        for (int i = tid; i < H * 9; i += L::kThreads) sK[i] = a.K[pod * H * 9 + i];
        for (int i = tid; i < H * H; i += L::kThreads) {
            const int hh = i / H, o = i % H;  // sMW[h][o] = M[o][h]
            sMW[i] = a.M[(pod * H + o) * H + hh];
        }
        if (tid < H) {
            sScale[tid] = a.scale_in ? a.scale_in[b * H + tid] : 1.0f;
            sScaleLo[tid] = a.scale_in ? a.scale_in[a.B * H + b * H + tid] : 0.0f;
            if (!a.per_cell) {
                const Growth gr = growth_args(a.growth_fn, a.mu[pod * H + tid], a.sigma[pod * H + tid], a.dt);
                sGa[tid] = gr.ga;
                sGb[tid] = gr.gb;
            }
        }
    }
    if (a.per_cell) {
        for (int i = tid; i < kTileCells * H; i += L::kThreads) {
            const int cell = i / H, h = i % H;
            const long long pi =
                (((long long)pod * G + ty0 + cell / kTileX) * G + tx0 + cell % kTileX) * H + h;
            sMS[(h * kTileCells + cell) * 2 + 0] = a.mu[pi];
            sMS[(h * kTileCells + cell) * 2 + 1] = a.sigma[pi];
        }
    }
    issue_head(0, bufA);

    // ---- phase-B task: a run of 4 cells of one tile row, two adjacent channels ----
    const bool active = tid < L::kActive;
    const int cp = tid % kPairs;
    const int grp = tid / kPairs;  // 0..7 when active
    const int ry = grp >> 1;
    const int rx0 = (grp & 1) * kRun;
    const int c0 = 2 * cp;
    // LDS byte offset of this thread's pair in halo cell (ry, rx0); a window column
    // moves by kRowB bytes, a window row by 10 kRowB.
    const int pbase = (ry * kHaloX + rx0) * L::kRowB + c0 * (int)sizeof(T);

    // ---- phase-A task: one cell, chunk group g of kTPC --------------------------------
    const int acell = tid / L::kTPC, ag = tid % L::kTPC;
    const int acy = acell / kTileX, acx = acell % kTileX;

    float y[H][kRun][2];
#pragma unroll
    for (int o = 0; o < H; ++o)
#pragma unroll
        for (int x = 0; x < kRun; ++x) y[o][x][0] = y[o][x][1] = 0.f;
    float xin[H] = {};

    const float inv_sqrt_d = 1.0f / __builtin_sqrtf((float)D);
    constexpr float kLog2e = 1.4426950408889634f;
    const Growth gc = growth_args(a.growth_fn, 0.f, 1.f, a.dt);  // c0, c1, c2 of the function

    auto do_head = [&](int h, const unsigned char* buf, unsigned char* nxt) {
        float* sA = sAtt[h & 1];
        wait_vm0();       // this wave's loads of head h have landed
        __syncthreads();  // ... and every other wave's; head h-1 is fully consumed
        if (h + 1 < H) issue_head(h + 1, nxt);

        // ---- phase A: attention scores (S4) and softmax --------------------------------
        {
            float s[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) s[k] = 0.f;
#pragma unroll
            for (int c = ag; c < L::kCPR; c += L::kTPC) {
                const uint4 pv = *reinterpret_cast<const uint4*>(
                    buf + L::offP + acell * L::kRowB + ((c ^ (acell & L::kSwz)) << 4));
#pragma unroll
                for (int k = 0; k < 9; ++k) {
                    const int nb = (acy + k / 3) * kHaloX + acx + k % 3;
                    const uint4 iv = *reinterpret_cast<const uint4*>(
                        buf + L::offI + nb * L::kRowB + ((c ^ (nb & L::kSwz)) << 4));
                    s[k] = chunk_dot<T>(pv, iv, s[k]);
                }
            }
            float m = -3.0e38f;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                s[k] = group_sum<L::kTPC>(s[k]) * inv_sqrt_d;
                m = fmaxf(m, s[k]);
            }
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                s[k] = exp2_fast((s[k] - m) * kLog2e);
                sum += s[k];
            }
            const float inv = 1.0f / sum;
            if (ag == 0) {
#pragma unroll
                for (int k = 0; k < 9; ++k) sA[acell * kAStride + k] = s[k] * inv;
            }
        }
        lds_barrier();

        // ---- phase B: potential, growth, propagation, update, head mixing --------------
        float xacc = 0.f;
        if (active) {
            const float s_in = sScale[h], s_lo = sScaleLo[h];
            float kw[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) kw[k] = sK[h * 9 + k];
            float mw[H];
#pragma unroll
            for (int o = 0; o < H; ++o) mw[o] = sMW[h * H + o];
            float ga = 0.f, gb = 0.f;
            if (!a.per_cell) {
                ga = sGa[h];
                gb = sGb[h];
            }
            const unsigned char* px = buf + L::offX + pbase;
            const unsigned char* pvv = buf + L::offV + pbase;

            float2 xw[3][3], vw[3][3];
#pragma unroll
            for (int dy = 0; dy < 3; ++dy)
#pragma unroll
                for (int dx = 0; dx < 2; ++dx) {
                    const int o = (dy * kHaloX + dx) * L::kRowB;
                    xw[dy][dx] = lds_pair<T>(px + o);
                    vw[dy][dx] = lds_pair<T>(pvv + o);
                }
#pragma unroll
            for (int x = 0; x < kRun; ++x) {
#pragma unroll
                for (int dy = 0; dy < 3; ++dy) {
                    const int o = (dy * kHaloX + x + 2) * L::kRowB;
                    xw[dy][2] = lds_pair<T>(px + o);
                    vw[dy][2] = lds_pair<T>(pvv + o);
                }
                const float* ap = sA + (ry * kTileX + rx0 + x) * kAStride;
                const float4 a0 = reinterpret_cast<const float4*>(ap)[0];
                const float4 a1 = reinterpret_cast<const float4*>(ap)[1];
                const float a8 = ap[8];
                const float aw[9] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w, a8};
                if (a.per_cell) {
                    const int cell = ry * kTileX + rx0 + x;
                    const float2 ms = *reinterpret_cast<const float2*>(sMS + (h * kTileCells + cell) * 2);
                    const Growth gr = growth_args(a.growth_fn, ms.x, ms.y, a.dt);
                    ga = gr.ga;
                    gb = gr.gb;
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
                    const float us = u * s_in;
                    const float tg = __builtin_fmaf(us, ga, -gb);
                    const float ex = exp2_fast(-tg * tg);
                    const float coef = __builtin_fmaf(ex, __builtin_fmaf(gc.c2, us, gc.c1), gc.c0);  // dt * g
                    const float xv = e ? xw[1][1].y : xw[1][1].x;
                    const float xc = __builtin_fmaf(xv, s_lo, xv * s_in);
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
                // Keep the scheduler from hoisting later cells' LDS reads over this
                // one: the output accumulators already take a large share of a
                // 2-waves-per-SIMD register budget.
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int j = 0; j < H; ++j) xin[j] = (j == h) ? xacc : xin[j];
    };
    for (int h = 0; h < H; h += 2) {
        do_head(h, bufA, bufB);
        do_head(h + 1, bufB, bufA);
    }

    // ---- phase C: store Y and the tile's mass partial sums ------------------------------
    TY* Yg = static_cast<TY*>(a.Y);
    float ysum[H];
#pragma unroll
    for (int o = 0; o < H; ++o) ysum[o] = 0.f;
    if (active) {
#pragma unroll
        for (int x = 0; x < kRun; ++x) {
            const long long base = bbase + ((long long)(ty0 + ry) * G + tx0 + rx0 + x) * C + c0;
#pragma unroll
            for (int o = 0; o < H; ++o) {
                const float r0 = Store<TY>::round(y[o][x][0]);
                const float r1 = Store<TY>::round(y[o][x][1]);
                ysum[o] += r0 + r1;
                Store<TY>::store2(Yg + base + o * D, r0, r1);
            }
        }
    }
    // Each lane's few values are summed in fp32; lanes, waves and tiles add in fp64,
    // so the sums stay accurate when the state's values are large and of both signs.
#pragma unroll
    for (int j = 0; j < H; ++j) {
        const double sx = wave_sum64(xin[j]);
        const double sy = wave_sum64(ysum[j]);
        if (lane == 0) {
            sR[wave * 16 + j] = sx;
            sR[wave * 16 + H + j] = sy;
        }
    }
    __syncthreads();
    if (tid < 2 * H) {
        double sum = 0.0;
        for (int w = 0; w < L::kWaves; ++w) sum += sR[w * 16 + tid];
        const int j = tid % H;
        double* dst = tid < H ? a.part_in : a.part_out;
        dst[((long long)b * H + j) * tpb + tile] = sum;
    }
}

// ---- bf16 state, D = 64: the neighbourhood sums on the matrix cores ------------------
//
// Same tiles and outputs as stencil_kernel, but S2 and S5 -- the two 9-tap sums per
// (cell, channel) that dominate the generic kernel's VALU work -- become MFMA
// products over the staged halo:
//   U^T  = X_halo^T . Kmat^T      Kmat[cell][n] = K[h][k] if halo row n = n_k(cell)
//   Vt^T = V_halo^T . Att^T       Att[cell][n]  = a_k(cell) likewise (0 elsewhere)
// (M = 16 channels, N = 16 cells, K = 64 halo rows; v_mfma_f32_16x16x32_bf16).
// Weights enter as bf16 hi + lo pairs (w = hi + lo to 2^-17 relative) and X, V
// are bf16 already, so every product is exact in fp32 and the sums keep fp32
// accuracy. The halo^T operands come straight from the row-major halo through
// ds_read_b64_tr_b16 (gfx950's transposing LDS read). Kmat depends only on the
// pod's 9 weights of the head and the tile geometry: each lane builds its Kmat^T
// operand with v_perm_b32 from a 12-dword table per (pod, head) that sits in the
// tile's parameter block (stencil_band.hpp), so the weights cost no vector-memory
// traffic; Att is built per head.
//
// Work split: wave w owns cell block cb = w/2 (tile rows 2cb, 2cb+1: 16 cells)
// and channel half w%2 (32 channels). Each wave computes the scores <P, I> of its
// 16 cells against the 48 halo rows that can hold their neighbours (matrix
// cores), keeps the 9 per cell, runs the softmax (4 lanes per cell) and writes
// Att for its cells into its own LDS region -- nothing crosses waves inside a
// head, so the only barrier per head is the one that publishes the staged halo.
// Growth, update and head mixing then run in registers for its 16 x 32 outputs.
//
// The kernel is persistent: a workgroup takes tiles of its XCD's eighth in order from
// the XCD's ticket counter (stencil_sched.hpp), and the staging pipeline runs across
// tile boundaries -- head 0 of the next tile and
// that tile's parameters are in flight while the last head of the current one
// computes -- so no workgroup starts from an empty pipeline.
namespace mf {

constexpr int kD = 64;
constexpr int kRowB = kD * 2;                          // bytes per (cell, head) row
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int offX = 0, offV = kHaloPad * kRowB, offI = 2 * kHaloPad * kRowB,
              offP = 3 * kHaloPad * kRowB;
constexpr int kBufB = (3 * kHaloPad + kTileCells) * kRowB;  // 28 KiB
constexpr int kWC = 16;                                     // cells per wave
constexpr int kAttB = kWC * kRowB;                          // one 16 x 64 bf16 matrix
constexpr int kS9 = 12;  // floats per cell in a score buffer (9 used, 9..11 take discards)
// Per-tile parameter block (fp32): M transposed (M[o][h] at h*8+o, so that head h's
// eight mixing weights are two 16-byte reads); per head h at kPH + 4h the deferred
// mass scale of X, its low part, mu and sigma (one 16-byte read); then, for per-cell
// growth, mu and sigma [cell][8]; then the pod's 3x3-kernel band table
// (stencil_band.hpp), 12 dwords per head.
constexpr int kPM = 0, kPH = 64, kPScal = 96;
constexpr int kPCellMu = 96, kPCellSg = 96 + kTileCells * 8, kPBand = 96 + 2 * kTileCells * 8;
constexpr int kBandHead = 12;                       // dwords per head: 3 runs x {A, B} x {hi, lo}
constexpr int kParF = kPBand + kHeads * kBandHead;
static_assert(kPBand % 4 == 0 && kPH % 4 == 0, "16-byte reads of the band table and the per-head values");

// 16-byte chunk swizzles inside a 128-byte row. X and V: any four consecutive
// rows 4j..4j+3, and rows {r, r+2, r+8, r+10}, occupy disjoint chunk pairs, so
// the transposing reads (4 rows x 32 bytes per 16 lanes) are free of bank
// conflicts. I and P: chunk ^ (row & 7).
__device__ __forceinline__ int swz_xv(int row) { return 2 * ((row ^ (row >> 3)) & 3); }
__device__ __forceinline__ int swz_ip(int row) { return row & 7; }

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4 of
// the 8 bytes read by lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4 (in that order).
__device__ __forceinline__ uint2 read_tr16(const unsigned char* p) {
    const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4i16*)(const __attribute__((address_space(3))) unsigned char*)(p));
    return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, a),
                                                  __builtin_bit_cast(bf16x8_v, b), c, 0, 0, 0);
}

// hi + lo bf16 split of an fp32 weight.
__device__ __forceinline__ void split_bf16(float v, bf16_t& hi, bf16_t& lo) {
    hi = f32_to_bf16(v);
    lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// One step of a butterfly sum of kN*2 per-lane values: lanes whose bit `bit` is
// set keep the upper half, the others the lower half, each adding the partner
// lane's copy (DPP kCtrl, whose partner differs from the lane in that bit and in
// no bit a previous step used).
template <int kN, int kCtrl>
__device__ __forceinline__ void fold_half(double (&v)[16], int lane, int bit) {
    const bool up = (lane >> bit) & 1;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
        const double keep = up ? v[i + kN] : v[i];
        const double send = up ? v[i] : v[i + kN];
        v[i] = keep + dpp_f64<kCtrl>(send);
    }
}

// Halo row of neighbour k of tile cell c (4 x 8 tile, 6 x 10 halo).
__host__ __device__ constexpr int nb_row(int c, int k) {
    return (c / kTileX + k / 3) * kHaloX + c % kTileX + k % 3;
}

}  // namespace mf

// kGrowthFn: false for the bell growth; true for any of the three growth functions
// through growth_args (one more multiply-add per value). kLoss (fp32 Y only): the
// backward's tape step, which also sums Y^2, Y T and T^2 per (b, head, tile).
template <typename TY, bool kGrowthFn, bool kLoss = false>
__global__ __launch_bounds__(mf::kThreads, 2) void stencil_mfma_kernel(StencilArgs a) {
    using namespace mf;
    constexpr int H = kHeads;
    constexpr int C = H * kD;
    __shared__ __attribute__((aligned(16))) unsigned char bufA[kBufB];
    __shared__ __attribute__((aligned(16))) unsigned char bufB[kBufB];
    // Per wave: Att of its 16 cells, [hi/lo][cell][halo row] bf16, chunk-swizzled
    // by cell & 7; and its 16 cells' 9 scores.
    __shared__ __attribute__((aligned(16))) unsigned char sAtt[kWaves * 2 * kAttB];
    __shared__ __attribute__((aligned(16))) float sS9[kWaves * kWC * kS9];
    // One parameter block: a tile's block is written after the barrier that ends
    // the previous tile's last head, its last reader.
    __shared__ __attribute__((aligned(16))) float sPar[kParF];
    __shared__ double sR[kThreads];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.G;
    const int tiles_x = G / kTileX;
    const int tpb = (G / kTileY) * tiles_x;
    const int ntiles = a.B * tpb;

    // ---- this workgroup's tiles (stencil_sched.hpp) -----------------------------------
    // Ticketed: the XCD's counter a.sched[x] hands out its eighth of the tiles in order
    // after the fixed first ones, so the tiles in flight on an XCD stay a window of
    // consecutive tiles, whose shared halo lines its L2 serves once: with a fixed
    // stride the workgroups drift apart over a launch and neighbours fetch the same
    // lines from HBM again (16 % more read traffic, 3 % more time at c3).
    // a.sched[8 + x] counts the XCD's finished workgroups; the last one zeroes both
    // counters for the next launch, which stream order puts after it.
    const sched::StencilWalk walk = sched::stencil_walk(blockIdx.x, gridDim.x, ntiles);
    const bool ticketed = walk.ticketed;
    int t_cur = walk.t_cur;
    if (!sched::has_tile(walk)) return;  // not one of the XCD's counted workgroups
    __shared__ int sTicket;

    const int cb = wave >> 1, chh = wave & 1;   // cell block, channel half
    const int grp = lane >> 4, i16 = lane & 15;
    const int cell = kWC * cb + i16;            // this lane's cell in phase B
    const unsigned* kband = static_cast<const unsigned*>(a.kband);

    // ---- staging: 8 halo rows (or P rows) per direct-load instruction -------------------
    // Lane l of an instruction lands at row g*8 + l/8, physical chunk l%8, and fetches
    // the logical chunk the row's swizzle maps there. Wave w issues groups w and w+4
    // of each halo array and group w of the P tile.
    unsigned boff_xv[2], boff_i[2], boff_p;
    const char *srcX, *srcV, *srcI, *srcP;
    auto set_tile = [&](int t) {  // per-lane offsets and bases of tile t
        const int b = t / tpb, tile = t % tpb;
        const int ty0 = (tile / tiles_x) * kTileY, tx0 = (tile % tiles_x) * kTileX;
        const int pc = lane & 7;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int row = (wave + 4 * k) * 8 + (lane >> 3);
            const int gc = row < kHaloCells ? row : kHaloCells - 1;  // padding rows
            const int gy = wrapi(ty0 + gc / kHaloX - 1, G), gx = wrapi(tx0 + gc % kHaloX - 1, G);
            const int base = (gy * G + gx) * C;
            boff_xv[k] = (unsigned)(base + (pc ^ swz_xv(row)) * 8) * 2u;
            boff_i[k] = (unsigned)(base + (pc ^ swz_ip(row)) * 8) * 2u;
        }
        const int row = wave * 8 + (lane >> 3);  // tile cell
        const int base = ((ty0 + row / kTileX) * G + tx0 + row % kTileX) * C;
        boff_p = (unsigned)(base + (pc ^ swz_ip(row)) * 8) * 2u;
        const long long bb = (long long)b * G * G * C;
        srcX = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.X) + bb);
        srcV = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.V) + bb);
        srcI = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.I) + bb);
        srcP = reinterpret_cast<const char*>(static_cast<const bf16_t*>(a.P) + bb);
    };
    auto issue_head = [&](int h, unsigned char* buf) {
        const unsigned hb = (unsigned)(h * kRowB);
        const unsigned lb = lds_addr(buf);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const unsigned row = lb + (wave + 4 * k) * 1024;
            dma16_lds(srcX, boff_xv[k] + hb, row + offX);
            dma16_lds(srcV, boff_xv[k] + hb, row + offV);
            dma16_lds(srcI, boff_i[k] + hb, row + offI);
        }
        dma16_lds_nt(srcP, boff_p + hb, lb + offP + wave * 1024);
    };
    // Per-tile parameters: up to four values per lane, loaded into registers with
    // the tile's first staging and written to LDS once they have landed.
    float pre[3];
    unsigned pre_band = 0u;
    auto fetch_params = [&](int t) {
        const int b = t / tpb, tile = t % tpb;
        const int pod = b / a.per_pod;
        pre[0] = pre[1] = pre[2] = 0.f;
        if (tid < H * kBandHead) pre_band = kband[pod * H * kBandHead + tid];
        if (tid < kPM + 64) {
            const int hh = (tid - kPM) >> 3, o = (tid - kPM) & 7;
            pre[0] = a.M[pod * 64 + o * 8 + hh];
        } else if (tid < kPScal) {
            const int hh = (tid - kPH) >> 2, f = (tid - kPH) & 3;
            if (f == 0) pre[0] = a.scale_in ? a.scale_in[b * 8 + hh] : 1.0f;
            else if (f == 1) pre[0] = a.scale_in ? a.scale_in[a.B * 8 + b * 8 + hh] : 0.0f;
            else if (!a.per_cell) pre[0] = f == 2 ? a.mu[pod * 8 + hh] : a.sigma[pod * 8 + hh];
        }
        if (a.per_cell) {
            const int ty0 = (tile / tiles_x) * kTileY, tx0 = (tile % tiles_x) * kTileX;
            const int pcell = tid >> 3, hh = tid & 7;
            const long long pi =
                (((long long)pod * G + ty0 + pcell / kTileX) * G + tx0 + pcell % kTileX) * H + hh;
            pre[1] = a.mu[pi];
            pre[2] = a.sigma[pi];
        }
    };
    auto store_params = [&](float* par) {
        if (tid < kPScal) par[tid] = pre[0];
        if (tid < H * kBandHead) reinterpret_cast<unsigned*>(par)[kPBand + tid] = pre_band;
        if (a.per_cell) {
            par[kPCellMu + tid] = pre[1];
            par[kPCellSg + tid] = pre[2];
        }
    };

    // Att is zero except at the 9 neighbours of each cell.
    for (int i = tid; i < kWaves * 2 * kAttB / 16; i += kThreads)
        reinterpret_cast<uint4*>(sAtt)[i] = make_uint4(0u, 0u, 0u, 0u);
    set_tile(t_cur);
    fetch_params(t_cur);
    issue_head(0, bufA);
    // Head 0's loads are always waited for before the head-0 barrier is reached (here
    // for the first tile, at the previous tile's end otherwise), so that barrier does
    // not wait for the previous tile's Y stores, the youngest memory operations then.
    // The empty statement marks the parameter registers as produced after that wait,
    // or the compiler adds a full wait for their loads at the head-0 barrier.
    wait_vm0();
    asm volatile("" : "+v"(pre[0]), "+v"(pre[1]), "+v"(pre[2]), "+v"(pre_band));

    // ---- per-lane roles (tile independent) ----------------------------------------------
    unsigned char* att = sAtt + wave * 2 * kAttB;
    float* s9 = sS9 + wave * kWC * kS9;
    // scores: A = P rows of cells 16 cb + i16, B = I rows of halo blocks j = cb .. cb+2
    // (the 48 halo rows holding the block's neighbours); K = channels.
    unsigned sp_off[2], si_off[3][2], s9_off[3][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        sp_off[ks] = (unsigned)(offP + cell * kRowB + (((4 * ks + grp) ^ swz_ip(cell)) << 4));
#pragma unroll
        for (int jj = 0; jj < 3; ++jj) {
            const int n = 16 * (cb + jj) + i16;
            si_off[jj][ks] = (unsigned)(offI + n * kRowB + (((4 * ks + grp) ^ swz_ip(n)) << 4));
        }
    }
#pragma unroll
    for (int jj = 0; jj < 3; ++jj)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // result (jj, e): cell kWC cb + 4 grp + e, halo row n = 16 (cb + jj) + i16
            const int lc = 4 * grp + e, c = kWC * cb + lc, n = 16 * (cb + jj) + i16;
            const int dy = n / kHaloX - c / kTileX, dx = n % kHaloX - c % kTileX;
            const bool keep = n < kHaloCells && (unsigned)dy < 3u && (unsigned)dx < 3u;
            s9_off[jj][e] = (unsigned)(lc * kS9 + (keep ? 3 * dy + dx : 9 + jj)) * 4u;
        }
    // softmax: 4 lanes per cell; lane q of cell sc takes neighbours q and q + 4,
    // lane 0 also neighbour 8.
    const int sc = lane >> 2, sq = lane & 3;
    auto wpos = [&](int k) {  // byte offset of (cell sc, neighbour k) in an Att matrix
        const int n = nb_row(kWC * cb + sc, k);
        return sc * kRowB + (((n >> 3) ^ (sc & 7)) << 4) + (n & 7) * 2;
    };
    const int wp_a = wpos(sq), wp_b = wpos(sq + 4), wp_8 = wpos(8);
    // phase B: channels 32 chh + 16 mb + 4 grp .. +3 (mb = 0, 1) of cell `cell`.
    unsigned tr_off[2][2][2];  // [mb][ks][hf]: halo row 32 ks + 8 grp + 4 hf + i16/4
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int row = 32 * ks + 8 * grp + 4 * hf + (i16 >> 2);
                const int cblk = 2 * chh + mb, q = i16 & 3;
                tr_off[mb][ks][hf] = (unsigned)(row * kRowB + (((2 * cblk + (q >> 1)) ^ swz_xv(row)) << 4) +
                                                8 * (q & 1));
            }
    unsigned at_off[2];  // Att^T operand: local cell i16, halo rows 32 ks + 8 grp .. +7
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) at_off[ks] = (unsigned)(i16 * kRowB + (((4 * ks + grp) ^ (i16 & 7)) << 4));
    unsigned xc_off[2];  // centre row of `cell`, channels 32 chh + 16 mb + 4 grp .. +3
    {
        const int crow = nb_row(cell, 4);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int cblk = 2 * chh + mb;
            xc_off[mb] = (unsigned)(offX + crow * kRowB + (((2 * cblk + (grp >> 1)) ^ swz_xv(crow)) << 4) +
                                    8 * (grp & 1));
        }
    }
    const int ch0 = 32 * chh + 4 * grp;  // + 16 mb: this lane's output channels
    // Kmat^T operand of this lane (cell, halo rows 32 ks + 8 grp .. +7): the band-table
    // run it meets (dword offset in a head's table) and the byte selectors of its dwords.
    unsigned band_row[2], band_sel[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        band_row[ks] = (unsigned)(4 * band::band_run(cell, grp, ks));
#pragma unroll
        for (int d = 0; d < 4; ++d) band_sel[ks][d] = band::band_sel(cell, grp, ks, d);
    }

    constexpr float kLog2e = 1.4426950408889634f;
    const float score_scale = kLog2e / 8.0f;  // log2(e) / sqrt(D)
    const float sqrt_log2e = __builtin_sqrtf(kLog2e);
    const float dt = a.dt;

    float y[H][2][4];
    float xin[H];
    int gh = 0;  // heads processed by this workgroup (selects the staging buffer)
    while (true) {
        // The next tile: fixed stride, or the ticket thread 0 draws after head 1's
        // barrier and publishes through LDS before the last head, which starts that
        // tile's loads.
        int ticket = 0;
        int t_next = ticketed ? -1 : sched::strided_next(walk, t_cur);
        const int b = t_cur / tpb, tile = t_cur % tpb;
        const int ty0 = (tile / tiles_x) * kTileY, tx0 = (tile % tiles_x) * kTileX;
        const long long bbase = (long long)b * G * G * C;
        float* par = sPar;
#pragma unroll
        for (int o = 0; o < H; ++o) {
            xin[o] = 0.f;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int e = 0; e < 4; ++e) y[o][mb][e] = 0.f;
        }

        for (int h = 0; h < H; ++h, ++gh) {
            const unsigned char* buf = (gh & 1) ? bufB : bufA;
            unsigned char* nxt = (gh & 1) ? bufA : bufB;
            if (h > 0) wait_vm0();  // this wave's loads of head h have landed
            __syncthreads();        // ... and every other wave's; head h-1 is fully consumed
            if (h == 0) store_params(par);
            // Drawn after head 1's barrier, when nothing else is in flight; written after
            // head 2's, whose wait has covered the draw, and read after head H-1's. The
            // next tile's write follows the tile-end barrier.
            if (ticketed && h == 1 && tid == 0) {
                // An address the compiler cannot prove uniform keeps the draw a plain
                // per-lane atomic, whose result is waited for at its use; as a uniform
                // one it is rewritten into a wave-wide form that waits at once.
                auto* ctr = (__attribute__((address_space(1))) unsigned*)(a.sched + walk.xcd);
                asm volatile("" : "+v"(ctr));
                ticket = (int)__hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (ticketed && h == 2 && tid == 0) sTicket = ticket;
            if (ticketed && h == H - 1) {
                t_next = sched::ticket_tile(walk, __builtin_amdgcn_readfirstlane(sTicket));
            }
            if (h + 1 < H) {
                issue_head(h + 1, nxt);
            } else if (t_next >= 0) {
                set_tile(t_next);
                fetch_params(t_next);
                issue_head(0, nxt);
            }

            // ---- S4 scores of this wave's cells, kept for the 9 neighbours --------------
            {
                // All operand reads first, then the MFMAs: the compiler would otherwise
                // reuse registers and wait for each read in turn.
                const uint4 pa0 = *reinterpret_cast<const uint4*>(buf + sp_off[0]);
                const uint4 pa1 = *reinterpret_cast<const uint4*>(buf + sp_off[1]);
                uint4 ib[3][2];
#pragma unroll
                for (int jj = 0; jj < 3; ++jj)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) ib[jj][ks] = *reinterpret_cast<const uint4*>(buf + si_off[jj][ks]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int jj = 0; jj < 3; ++jj) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    acc = mfma16(pa0, ib[jj][0], acc);
                    acc = mfma16(pa1, ib[jj][1], acc);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        *reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(s9) + s9_off[jj][e]) =
                            acc[e];
                }
            }
            // ---- S2: U = X_halo^T . Kmat^T on the matrix cores. It does not depend on the
            // softmax, so its operand reads and MFMAs go first and overlap that chain.
            uint4 kq[2][2];  // Kmat^T [ks][hi/lo], from the head's band-table run
            {
                const unsigned* kb = reinterpret_cast<const unsigned*>(par) + kPBand + h * kBandHead;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const uint4 t = *reinterpret_cast<const uint4*>(kb + band_row[ks]);  // A, B hi; A, B lo
                    kq[ks][0] = make_uint4(__builtin_amdgcn_perm(t.y, t.x, band_sel[ks][0]),
                                           __builtin_amdgcn_perm(t.y, t.x, band_sel[ks][1]),
                                           __builtin_amdgcn_perm(t.y, t.x, band_sel[ks][2]),
                                           __builtin_amdgcn_perm(t.y, t.x, band_sel[ks][3]));
                    kq[ks][1] = make_uint4(__builtin_amdgcn_perm(t.w, t.z, band_sel[ks][0]),
                                           __builtin_amdgcn_perm(t.w, t.z, band_sel[ks][1]),
                                           __builtin_amdgcn_perm(t.w, t.z, band_sel[ks][2]),
                                           __builtin_amdgcn_perm(t.w, t.z, band_sel[ks][3]));
                }
            }
            // The 16 transposing reads of X and V first (both are needed below).
            uint4 ax[2][2], av[2][2];  // [mb][ks]
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const uint2 x0 = read_tr16(buf + offX + tr_off[mb][ks][0]);
                    const uint2 x1 = read_tr16(buf + offX + tr_off[mb][ks][1]);
                    const uint2 v0 = read_tr16(buf + offV + tr_off[mb][ks][0]);
                    const uint2 v1 = read_tr16(buf + offV + tr_off[mb][ks][1]);
                    ax[mb][ks] = make_uint4(x0.x, x0.y, x1.x, x1.y);
                    av[mb][ks] = make_uint4(v0.x, v0.y, v1.x, v1.y);
                }
            __builtin_amdgcn_sched_barrier(0);
            f32x4 u[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                u[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int m = 0; m < 2; ++m) u[mb] = mfma16(ax[mb][ks], kq[ks][m], u[mb]);
            }
            // ---- softmax; Att of this wave's cells (its own LDS: in order, no barrier) -
            {
                const float* srow = s9 + sc * kS9;
                const float s_a = srow[sq], s_b = srow[sq + 4], s_8 = srow[8];
                const float m_l = sq == 0 ? fmaxf(fmaxf(s_a, s_b), s_8) : fmaxf(s_a, s_b);
                const float mx = group_max<4>(m_l);
                const float e_a = exp2_fast((s_a - mx) * score_scale);
                const float e_b = exp2_fast((s_b - mx) * score_scale);
                const float e_8 = exp2_fast((s_8 - mx) * score_scale);
                const float inv = rcp_fast(group_sum<4>(sq == 0 ? e_a + e_b + e_8 : e_a + e_b));
                bf16_t hi, lo;
                split_bf16(e_a * inv, hi, lo);
                *reinterpret_cast<bf16_t*>(att + wp_a) = hi;
                *reinterpret_cast<bf16_t*>(att + kAttB + wp_a) = lo;
                split_bf16(e_b * inv, hi, lo);
                *reinterpret_cast<bf16_t*>(att + wp_b) = hi;
                *reinterpret_cast<bf16_t*>(att + kAttB + wp_b) = lo;
                if (sq == 0) {
                    split_bf16(e_8 * inv, hi, lo);
                    *reinterpret_cast<bf16_t*>(att + wp_8) = hi;
                    *reinterpret_cast<bf16_t*>(att + kAttB + wp_8) = lo;
                }
            }

            // ---- S3 from U, then S5 on the matrix cores, S6 and head mixing --------------
            {
                // S3 and the scaled X need only U and the parameters: they run while the
                // Att values land and the S5 MFMAs work; exp2 over all 8 values at once.
                const float4 ph = *reinterpret_cast<const float4*>(par + kPH + 4 * h);
                const float s_in = ph.x, s_lo = ph.y;  // deferred mass scale of X, high and low parts
                const float two_dt = 2.0f * dt;
                float mw[H];
                {
                    const float4 m0 = *reinterpret_cast<const float4*>(par + kPM + h * H);
                    const float4 m1 = *reinterpret_cast<const float4*>(par + kPM + h * H + 4);
                    mw[0] = m0.x, mw[1] = m0.y, mw[2] = m0.z, mw[3] = m0.w;
                    mw[4] = m1.x, mw[5] = m1.y, mw[6] = m1.z, mw[7] = m1.w;
                }
                // (U s - mu) / (sigma + 1e-7) * sqrt(log2 e) = U ga - gb
                const float mu_h = a.per_cell ? par[kPCellMu + cell * 8 + h] : ph.z;
                const float sg_h = a.per_cell ? par[kPCellSg + cell * 8 + h] : ph.w;
                float ga, gb, c0 = -dt, c1 = two_dt, c2s = 0.f;
                if constexpr (kGrowthFn) {
                    const Growth gr = growth_args(a.growth_fn, mu_h, sg_h, dt);
                    ga = gr.ga * s_in, gb = gr.gb;
                    c0 = gr.c0, c1 = gr.c1, c2s = gr.c2 * s_in;  // c2 multiplies the scaled U
                } else {
                    const float gsc = sqrt_log2e / (sg_h + 1e-7f);
                    ga = gsc * s_in, gb = mu_h * gsc;
                }
                float coef[2][4], xcs[2][4], ex[2][4];  // dt * g, scaled X, bell argument
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float tg = __builtin_fmaf(u[mb][e], ga, -gb);
                        ex[mb][e] = -tg * tg;
                    }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) ex[mb][e] = exp2_fast(ex[mb][e]);
                float xacc = 0.f;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const uint2 xr = *reinterpret_cast<const uint2*>(buf + xc_off[mb]);
                    const float xv[4] = {bf16lo(xr.x), bf16hi(xr.x), bf16lo(xr.y), bf16hi(xr.y)};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (kGrowthFn)
                            coef[mb][e] = __builtin_fmaf(ex[mb][e], __builtin_fmaf(c2s, u[mb][e], c1), c0);
                        else
                            coef[mb][e] = __builtin_fmaf(ex[mb][e], two_dt, -dt);
                        xcs[mb][e] = __builtin_fmaf(xv[e], s_lo, xv[e] * s_in);
                        xacc += xcs[mb][e];
                    }
                }
                uint4 aw[2][2];  // Att^T [ks][hi/lo]
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int m = 0; m < 2; ++m)
                        aw[ks][m] = *reinterpret_cast<const uint4*>(att + m * kAttB + at_off[ks]);
                f32x4 vt[2];
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    vt[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int m = 0; m < 2; ++m) vt[mb] = mfma16(av[mb][ks], aw[ks][m], vt[mb]);
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float z = __builtin_fmaf(coef[mb][e], vt[mb][e], xcs[mb][e]);
#pragma unroll
                        for (int o = 0; o < H; ++o) y[o][mb][e] = __builtin_fmaf(mw[o], z, y[o][mb][e]);
                    }
#pragma unroll
                for (int j = 0; j < H; ++j) xin[j] = (j == h) ? xacc : xin[j];
            }
        }

        // ---- store Y and the tile's mass partial sums -----------------------------------
        // The next tile's parameters and head-0 loads have had the last head to land.
        wait_vm0();
        asm volatile("" : "+v"(pre[0]), "+v"(pre[1]), "+v"(pre[2]), "+v"(pre_band));
        TY* Yg = static_cast<TY*>(a.Y);
        float ysum[H];  // this lane's sum of stored Y per head
        double lsum[3][kLoss ? H : 1];  // kLoss: this lane's Y^2, Y T, T^2 per head
#pragma unroll
        for (int o = 0; o < H; ++o) ysum[o] = 0.f;
        if constexpr (kLoss) {
#pragma unroll
            for (int o = 0; o < H; ++o) lsum[0][o] = lsum[1][o] = lsum[2][o] = 0.0;
        }
        if constexpr (sizeof(TY) == 2) {
            // bf16: lanes grp and grp ^ 1 (lane ^ 16, the same cell) exchange one
            // 8-byte piece per head so that each stores 8 contiguous channels in one
            // 16-byte store -- even grp the mb = 0 block's, odd grp the mb = 1 block's
            // -- halving the store instructions of the tile. v_permlane16_swap(a, b)
            // swaps the odd 16-lane rows of a with the even rows of b; with a = the
            // mb = 0 piece and b = the mb = 1 piece, an even-row lane l is left with
            // (a[l], a[l + 16]) and an odd-row lane with (b[l - 16], b[l]), which is
            // that lane's 16 bytes in channel order.
            const long long base = bbase + ((long long)(ty0 + cell / kTileX) * G + tx0 + cell % kTileX) * C +
                                   32 * chh + 16 * (grp & 1) + 8 * (grp >> 1);
#pragma unroll
            for (int o = 0; o < H; ++o) {
                uint2 pk[2];
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    float r[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        r[e] = Store<TY>::round(y[o][mb][e]);
                        ysum[o] += r[e];
                    }
                    pk[mb] = make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
                }
                const auto sx = __builtin_amdgcn_permlane16_swap(pk[0].x, pk[1].x, false, false);
                const auto sy = __builtin_amdgcn_permlane16_swap(pk[0].y, pk[1].y, false, false);
                *reinterpret_cast<uint4*>(Yg + base + o * kD) = make_uint4(sx[0], sy[0], sx[1], sy[1]);
            }
        } else {
            const long long base =
                bbase + ((long long)(ty0 + cell / kTileX) * G + tx0 + cell % kTileX) * C + ch0;
            // kLoss: the target at this lane's 4 x 2 channels of every head, all loads
            // issued before the stores
            uint2 tw[kLoss ? 2 : 1][kLoss ? H : 1];
            if constexpr (kLoss) {
                const bf16_t* Tg = static_cast<const bf16_t*>(a.T);
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int o = 0; o < H; ++o)
                        tw[mb][o] = *reinterpret_cast<const uint2*>(Tg + base + o * kD + 16 * mb);
            }
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int o = 0; o < H; ++o) {
                    float r[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        r[e] = Store<TY>::round(y[o][mb][e]);
                        ysum[o] += r[e];
                    }
                    if constexpr (kLoss) {
                        // products of an fp32 and a bf16 value are exact in fp64
                        const float t4[4] = {bf16lo(tw[mb][o].x), bf16hi(tw[mb][o].x), bf16lo(tw[mb][o].y),
                                             bf16hi(tw[mb][o].y)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const double yd = r[e], td = t4[e];
                            lsum[0][o] = __builtin_fma(yd, yd, lsum[0][o]);
                            lsum[1][o] = __builtin_fma(yd, td, lsum[1][o]);
                            lsum[2][o] = __builtin_fma(td, td, lsum[2][o]);
                        }
                    }
                    // fp32: 16-byte pieces per cell, plain stores, so L2 merges the
                    // pieces of each 128-byte line before it is written back.
                    *reinterpret_cast<float4*>(Yg + base + o * kD + 16 * mb) = make_float4(r[0], r[1], r[2], r[3]);
                }
        }
        // Wave sums of the 16 values: the butterfly leaves lane l holding its 16-lane
        // row's sum of value l & 15; the rows and waves are added in a fixed order.
        // Each lane's 8 values per head are summed in fp32, everything above in fp64,
        // so the sums stay accurate when the state's values are large and of both signs.
        double red[16];  // [0, 8): sum of scaled X per head; [8, 16): sum of stored Y
#pragma unroll
        for (int o = 0; o < H; ++o) {
            red[o] = xin[o];
            red[H + o] = ysum[o];
        }
        fold_half<8, 0x140>(red, lane, 3);  // row_mirror: partner l ^ 15
        fold_half<4, 0x141>(red, lane, 2);  // row_half_mirror: partner l ^ 7
        fold_half<2, 0x4E>(red, lane, 1);   // quad_perm [2,3,0,1]: partner l ^ 2
        fold_half<1, 0xB1>(red, lane, 0);   // quad_perm [1,0,3,2]: partner l ^ 1
        sR[tid] = red[0];
        __syncthreads();
        if (tid < 2 * H) {
            double sum = 0.0;
#pragma unroll
            for (int r = 0; r < kThreads / 16; ++r) sum += sR[r * 16 + tid];
            const int j = tid % H;
            double* dst = tid < H ? a.part_in : a.part_out;
            dst[((long long)b * H + j) * tpb + tile] = sum;
        }
        if constexpr (kLoss) {
            // The same butterflies over [Y^2 | Y T] and [T^2 | 0], the rows added through
            // the last head's staging buffer: every wave has finished that head (the
            // barrier above), the next tile's first loads fill the other buffer, and
            // its first barrier follows these reads.
            double r2[16], r3[16];
#pragma unroll
            for (int o = 0; o < H; ++o) {
                r2[o] = lsum[0][o];
                r2[H + o] = lsum[1][o];
                r3[o] = lsum[2][o];
                r3[H + o] = 0.0;
            }
            fold_half<8, 0x140>(r2, lane, 3);
            fold_half<4, 0x141>(r2, lane, 2);
            fold_half<2, 0x4E>(r2, lane, 1);
            fold_half<1, 0xB1>(r2, lane, 0);
            fold_half<8, 0x140>(r3, lane, 3);
            fold_half<4, 0x141>(r3, lane, 2);
            fold_half<2, 0x4E>(r3, lane, 1);
            fold_half<1, 0xB1>(r3, lane, 0);
            double* scr = reinterpret_cast<double*>(((gh - 1) & 1) ? bufB : bufA);
            scr[tid] = r2[0];
            scr[kThreads + tid] = r3[0];
            __syncthreads();
            if (tid < 3 * H) {
                const int q = tid / H, j = tid % H;  // q: 0 Y^2, 1 Y T, 2 T^2
                const double* src = scr + (q == 2 ? kThreads : 0) + (q == 1 ? H : 0) + j;
                double sum = 0.0;
#pragma unroll
                for (int r = 0; r < kThreads / 16; ++r) sum += src[r * 16];
                a.loss_part[(((long long)b * H + j) * tpb + tile) * 3 + q] = sum;
            }
        }
        if (t_next < 0) break;
        t_cur = t_next;
    }
    // Every draw of this workgroup has returned (the last one ended the loop), so the
    // last of the XCD's counted workgroups to count itself here resets the counters.
    if (ticketed && tid == 0 &&
        sched::last_finisher(walk, __hip_atomic_fetch_add(a.sched + 8 + walk.xcd, 1u, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT))) {
        __hip_atomic_store(a.sched + walk.xcd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.sched + 8 + walk.xcd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <typename T, int D, typename TY>
hipError_t launch_tdy(const StencilArgs& a, hipStream_t s) {
    using L = Layout<T, D>;
    const int tiles = (a.G / kTileY) * (a.G / kTileX);
    hipLaunchKernelGGL((stencil_kernel<T, D, TY>), dim3(a.B * tiles), dim3(L::kThreads), 0, s, a);
    return hipGetLastError();
}

template <typename TY>
hipError_t launch_mfma(const StencilArgs& a, hipStream_t s) {
    int n_cu = 0;
    if (hipError_t e = device_cu_count(&n_cu); e != hipSuccess) return e;
    const int tiles = a.B * (a.G / kTileY) * (a.G / kTileX);
    const int grid = tiles < 2 * n_cu ? tiles : 2 * n_cu;  // two persistent workgroups per CU
    if (!a.sched) return hipErrorInvalidValue;
    if (a.T) {  // the backward's tape step: fp32 Y and the bell growth only
        if constexpr (std::is_same_v<TY, float>) {
            if (a.growth_fn != 0 || !a.loss_part) return hipErrorInvalidValue;
            hipLaunchKernelGGL((stencil_mfma_kernel<float, false, true>), dim3(grid), dim3(mf::kThreads), 0, s, a);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (a.growth_fn == 0)
        hipLaunchKernelGGL((stencil_mfma_kernel<TY, false>), dim3(grid), dim3(mf::kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((stencil_mfma_kernel<TY, true>), dim3(grid), dim3(mf::kThreads), 0, s, a);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_td(const StencilArgs& a, hipStream_t s) {
    if constexpr (sizeof(T) == 2 && D == 64)
        return a.y_f32 ? launch_mfma<float>(a, s) : launch_mfma<bf16_t>(a, s);
    else
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

size_t stencil_kband_bytes(int pods) { return (size_t)pods * kHeads * mf::kBandHead * 4; }

namespace {
// fp32 -> bf16 bits, round to nearest even (finite inputs).
uint16_t host_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float host_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
}  // namespace

void fill_stencil_kband(const float* K, int pods, uint32_t* out) {
    for (int p = 0; p < pods; ++p)
        for (int h = 0; h < kHeads; ++h) {
            const float* k = K + (p * kHeads + h) * 9;
            uint32_t* t = out + (size_t)(p * kHeads + h) * mf::kBandHead;
            for (int r = 0; r < 3; ++r) {
                uint16_t hi[3], lo[3];
                for (int q = 0; q < 3; ++q) {
                    hi[q] = host_bf16(k[3 * r + q]);
                    lo[q] = host_bf16(k[3 * r + q] - host_f32(hi[q]));
                }
                t[4 * r + 0] = hi[0] | (uint32_t)hi[1] << 16;  // A_hi
                t[4 * r + 1] = hi[2];                          // B_hi
                t[4 * r + 2] = lo[0] | (uint32_t)lo[1] << 16;  // A_lo
                t[4 * r + 3] = lo[2];                          // B_lo
            }
        }
}

hipError_t launch_stencil(int dtype, const StencilArgs& a, hipStream_t s) {
    return dtype == 1 ? launch_t<bf16_t>(a, s) : launch_t<float>(a, s);
}

}  // namespace slime
