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

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

__device__ __forceinline__ void wait_vm0() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // s_waitcnt vmcnt(0)
}

__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const lds_void_t*)p;
}

// One direct global->LDS load (global_load_lds_dwordx4, SGPR base + 32-bit lane
// offset): 16 bytes per lane from base + voff land at LDS byte address
// lds + 16 * lane. Issued through inline asm so that the per-lane addresses stay
// 32-bit (no 64-bit pointer per load held across the head loop); the kernel
// waits for these loads itself (wait_vm0) before the barrier that publishes them.
__device__ __forceinline__ void dma16_saddr(const void* base, unsigned voff, unsigned lds) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(lds), "v"(voff), "s"(base)
        : "memory", "m0");
}

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

// Score matrix of the MFMA score phase: 32 tile cells x 64 halo rows, fp32, rows
// padded to 72 floats so the two half-waves of an MFMA result write (rows m and
// m+4) land in different banks.
constexpr int kScoreLd = 72;

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
    // bf16, D = 64 (256 threads, 8 per cell): the scores <P, I> of all 32 cells
    // against all 64 staged halo rows come from the matrix cores (v_mfma
    // 32x32x16), 9 of each row are used.
    constexpr bool kMfmaScores = sizeof(T) == 2 && D == 64;
    __shared__ __attribute__((aligned(16))) float sS[kMfmaScores ? kTileCells * kScoreLd : 1];
    __shared__ __attribute__((aligned(16))) float sMS[H * kTileCells * 2];
    __shared__ float sR[L::kWaves * 16];

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
            dma16_saddr(srcX, boff_lin[k] + hb, row + L::offX);
            dma16_saddr(srcV, boff_lin[k] + hb, row + L::offV);
            dma16_saddr(srcI, boff_swz[k] + hb, row + L::offI);
        }
#pragma unroll
        for (int k = 0; k < L::kPA; ++k)
            dma16_saddr(srcP, boff_p[k] + hb, lds_addr(buf) + L::offP + (wave + k * L::kWaves) * 1024);
    };

    // Per-head parameters (and per-cell growth parameters) go to LDS once, before
    // any direct load is issued: reading them later from global memory would make
    // the in-order vector-memory counter wait for the next head's staging.
    __shared__ float sK[H * 9], sMW[H * H], sGa[H], sGb[H], sScale[H];
    {
        constexpr float kLog2eP = 1.4426950408889634f;
        for (int i = tid; i < H * 9; i += L::kThreads) sK[i] = a.K[pod * H * 9 + i];
        for (int i = tid; i < H * H; i += L::kThreads) {
            const int hh = i / H, o = i % H;  // sMW[h][o] = M[o][h]
            sMW[i] = a.M[(pod * H + o) * H + hh];
        }
        if (tid < H) {
            sScale[tid] = a.scale_in ? a.scale_in[b * H + tid] : 1.0f;
            if (!a.per_cell) {
                const float ga = __builtin_sqrtf(kLog2eP) / (a.sigma[pod * H + tid] + 1e-7f);
                sGa[tid] = ga;
                sGb[tid] = a.mu[pod * H + tid] * ga;
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
    const float sqrt_log2e = __builtin_sqrtf(kLog2e);

    auto do_head = [&](int h, const unsigned char* buf, unsigned char* nxt) {
        float* sA = sAtt[h & 1];
        wait_vm0();       // this wave's loads of head h have landed
        __syncthreads();  // ... and every other wave's; head h-1 is fully consumed
        if (h + 1 < H) issue_head(h + 1, nxt);

        // ---- phase A: attention scores (S4) and softmax --------------------------------
        if constexpr (kMfmaScores) {
            // Waves 0 and 1: S[cell][n] = <P_cell, I_n> for halo rows n of block 32*wave,
            // K = D channels in steps of 16. A = P (row = cell), B = I^T (column = halo
            // row); both operands are 16-byte chunks of swizzled rows.
            if (wave < 2) {
                const int m = lane & 31, kh = lane >> 5;
                const int n = 32 * wave + m;
                f32x16 acc = {};
#pragma unroll
                for (int ks = 0; ks < D / 16; ++ks) {
                    const int c = 2 * ks + kh;
                    const uint4 pa = *reinterpret_cast<const uint4*>(
                        buf + L::offP + m * L::kRowB + ((c ^ (m & L::kSwz)) << 4));
                    const uint4 ib = *reinterpret_cast<const uint4*>(
                        buf + L::offI + n * L::kRowB + ((c ^ (n & L::kSwz)) << 4));
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_v, pa),
                                                                  __builtin_bit_cast(bf16x8_v, ib), acc,
                                                                  0, 0, 0);
                }
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    sS[(8 * (e >> 2) + 4 * kh + (e & 3)) * kScoreLd + n] = acc[e];
            }
            lds_barrier();
            // Softmax over the 9 neighbours: 8 lanes per cell, lane j takes neighbour j,
            // lane 0 also neighbour 8.
            const int cell = tid >> 3, j = tid & 7;
            const int cy = cell / kTileX, cx = cell % kTileX;
            const float* srow = sS + cell * kScoreLd;
            const float sj = srow[(cy + j / 3) * kHaloX + cx + j % 3];
            const float s8 = srow[(cy + 2) * kHaloX + cx + 2];
            const float sc = inv_sqrt_d * kLog2e;
            float mx = group_max<8>(j == 0 ? fmaxf(sj, s8) : sj);
            const float ej = exp2_fast((sj - mx) * sc);
            const float e8 = exp2_fast((s8 - mx) * sc);
            const float inv = 1.0f / group_sum<8>(j == 0 ? ej + e8 : ej);
            sA[cell * kAStride + j] = ej * inv;
            if (j == 0) sA[cell * kAStride + 8] = e8 * inv;
        } else {
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
            const float s_in = sScale[h];
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
            const float dt = a.dt, two_dt = 2.0f * a.dt;
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
                    ga = sqrt_log2e / (ms.y + 1e-7f);
                    gb = ms.x * ga;
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
                    const float tg = __builtin_fmaf(u * s_in, ga, -gb);
                    const float ex = exp2_fast(-tg * tg);
                    const float coef = __builtin_fmaf(ex, two_dt, -dt);  // dt * g
                    const float xc = (e ? xw[1][1].y : xw[1][1].x) * s_in;
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
        float sum = 0.f;
        for (int w = 0; w < L::kWaves; ++w) sum += sR[w * 16 + tid];
        const int j = tid % H;
        float* dst = tid < H ? a.part_in : a.part_out;
        dst[((long long)b * H + j) * tpb + tile] = sum;
    }
}

template <typename T, int D, typename TY>
hipError_t launch_tdy(const StencilArgs& a, hipStream_t s) {
    using L = Layout<T, D>;
    const int tiles = (a.G / kTileY) * (a.G / kTileX);
    hipLaunchKernelGGL((stencil_kernel<T, D, TY>), dim3(a.B * tiles), dim3(L::kThreads), 0, s, a);
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
