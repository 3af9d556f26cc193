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
// frees the stage of slab k. Stages are laid out in fragment order (each MFMA
// operand read is one linear 1 KiB block: no bank conflicts). The first MFMA of
// a tile starts from a zero accumulator instead of clearing 256 registers. The
// weights are the MFMA "A" operand: a lane's accumulators hold 4 consecutive
// output channels of one cell. The bf16 epilogue goes through LDS so that stores
// leave as whole 128-byte row segments. Workgroups walk an XCD-contiguous tile
// range, N fastest, so a cell block and one batch's weights are re-read from that
// XCD's L2.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace slime {
namespace {


constexpr int kBM = 256, kBN = 256, kThreads = 256;
constexpr int kSlabB = 64;                    // bytes of K per tile row per slab
constexpr int kStageB = (kBM + kBN) * kSlabB;  // 32 KiB
constexpr int kDmaPerSlab = 8;                // direct-load instructions per wave per slab

// Stage layout: tile row r (0..255 cells, 256..511 output channels) holds its 64
// slab bytes at r*64, as four 16-byte chunks XOR-permuted by
// f(r) = ((r >> 1) ^ (r >> 3)) & 3: physical chunk = logical chunk ^ f(r). One
// direct-load instruction fills 16 whole rows (1 KiB, four lanes per 64-byte row),
// and the operand reads -- 32 consecutive rows at one logical chunk per half
// wave -- spread over the LDS banks.
__device__ __forceinline__ constexpr int row_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

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

// Marks an accumulator block as (re)defined in accumulator registers here, so the
// copies to vector registers that the epilogue needs are made next to their uses
// instead of all 256 right after the last MFMA.
__device__ __forceinline__ void pin_acc(f32x16& a) { asm volatile("" : "+a"(a)); }

// fp32 epilogue: direct 16-byte stores of 4 consecutive channels per lane.
template <int kAct>
__device__ __forceinline__ void store_tile_f32(f32x16 (&acc)[4][4], float* obase, int ncol) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float* orow = obase + (long long)j * 32 * ncol;
#pragma unroll
        for (int i = 0; i < 4; ++i) pin_acc(acc[i][j]);
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

// Rows of the per-wave staging region are padded to 144 bytes: the 8-byte writes
// of 16 consecutive rows hit distinct banks.
constexpr int kEpiRowB = 144;
constexpr int kEpiWaveB = 32 * kEpiRowB;
constexpr int kStoresBf16 = 32;  // global stores per wave per tile (bf16 epilogue)

typedef __attribute__((address_space(3))) void lds_void_t;

// One direct global->LDS load (global_load_lds_dwordx4, SGPR base + 32-bit lane
// offset): 16 bytes per lane from base + voff land at LDS byte address
// lds_base + 16 * lane. Issued through inline asm: the compiler would otherwise
// make every later LDS read wait for all such loads still in flight (it cannot
// tell which stage they fill). The pipeline waits for each slab itself (wait_vm)
// before the barrier that publishes it.
__device__ __forceinline__ void dma16(const void* base, unsigned voff, unsigned lds_base) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(lds_base), "v"(voff), "s"(base)
        : "memory", "m0");
}

__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const lds_void_t*)p;
}

// Issues the direct global->LDS loads of slab ks of a tile into the stage at LDS
// byte address sbase: 32 instructions of 16 rows each; wave w issues row groups
// w, w+4, ..., w+28 (16 cell groups, then 16 weight groups). x, w: the tile's
// first cell row and first weight row (uniform); voff: this lane's byte offset
// (row lane/4 of the group, the logical chunk that lands in physical chunk lane%4).
__device__ __forceinline__ void issue_slab(const char* x, const char* w, long long row_bytes, int ks,
                                           int wave, unsigned voff, unsigned sbase) {
    const long long k_off = (long long)ks * kSlabB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int grp = 4 * j + wave;
        dma16(x + grp * 16 * row_bytes + k_off, voff, sbase + grp * 1024);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int grp = 4 * j + wave;
        dma16(w + grp * 16 * row_bytes + k_off, voff, sbase + (16 + grp) * 1024);
    }
}

// s_waitcnt vmcnt(n) for the counts the pipeline needs (immediate operand).
__device__ __forceinline__ void wait_vm(int n) {
    // simm16: vmcnt[3:0] | expcnt(7)[6:4] | lgkmcnt(15)[11:8] | vmcnt[5:4] at [15:14]
#define SLIME_VMCNT(n) ((((n) & 15) | ((((n) >> 4) & 3) << 14)) | 0x0F70)
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(0)); break;
        case 8: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(8)); break;
        case 16: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(16)); break;
        case 24: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(24)); break;
        case 32: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(32)); break;
        case 40: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(40)); break;
        case 48: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(48)); break;
        default: __builtin_amdgcn_s_waitcnt(SLIME_VMCNT(0)); break;
    }
#undef SLIME_VMCNT
}

// Workgroup barrier for LDS data only: __syncthreads() would also wait for every
// outstanding vector-memory operation (its release fence covers the direct loads
// of later slabs and the previous tile's stores), draining the pipeline.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // s_waitcnt lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Operand fragments of one slab for one wave: weights (A operand, 4 blocks of 32
// output channels) and cells (B operand, 4 blocks of 32 cells), per 32-byte half kk.
struct Frags {
    u32x4 w[2][4];
    u32x4 x[2][4];
};

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Per-lane LDS byte offsets of this wave's fragments inside a stage, per half kk:
// x = its first cell row block, w = its first weight row block (row lane%32,
// physical chunk of logical chunk 2*kk + lane/32).
struct FragBase {
    unsigned x[2], w[2];
};

// Fragment read R (0..15) of the slab in the stage at `stage`, in the order the
// MFMAs consume them: per half kk, the 4 cell blocks then the 4 weight blocks
// (block q = 32 rows further).
template <int R>
__device__ __forceinline__ void read_frag(Frags& f, const unsigned char* stage, const FragBase& b) {
    constexpr int kk = R >> 3, q = R & 7;
    if constexpr (q < 4)
        f.x[kk][q] = *reinterpret_cast<const u32x4*>(stage + b.x[kk] + q * 32 * kSlabB);
    else
        f.w[kk][q - 4] = *reinterpret_cast<const u32x4*>(stage + b.w[kk] + (q - 4) * 32 * kSlabB);
}

// MFMA group M (0..31) of a slab: output block (i, j) = ((M / 4) % 4, M % 4) over
// half kk = M / 16; one bf16 MFMA or four fp32 MFMAs. kZero: start from 0.
template <typename T, bool kZero, int M>
__device__ __forceinline__ void mfma_group(f32x16 (&acc)[4][4], const Frags& f) {
    constexpr int kk = M >> 4, i = (M >> 2) & 3, j = M & 3;
    f32x16 c = acc[i][j];
    if constexpr (kZero) c = f32x16{};
    if constexpr (sizeof(T) == 2) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_v, f.w[kk][i]),
                                                            __builtin_bit_cast(bf16x8_v, f.x[kk][j]), c,
                                                            0, 0, 0);
    } else {
        const f32x4 wv = __builtin_bit_cast(f32x4, f.w[kk][i]);
        const f32x4 xv = __builtin_bit_cast(f32x4, f.x[kk][j]);
        f32x16 a = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[0], xv[0], c, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[1], xv[1], a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[2], xv[2], a, 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[3], xv[3], a, 0, 0, 0);
    }
}

// The tile/slab schedule a workgroup follows: persistent, each workgroup walks
// tiles tile, tile + stride, ... below tile_end (an XCD-contiguous range).
struct Walk {
    int tile, next, stride, tile_end, nN, nk;
    long long row_bytes;
    unsigned voff;              // this lane's byte offset within a 16-row load group
    const char *x_cur, *w_cur;  // this tile's first operand rows
    const char *x_nxt, *w_nxt;  // the next tile's, or this tile's when it is the last
};

// First operand rows of a tile (uniform across the workgroup).
template <typename T>
__device__ __forceinline__ void tile_rows(const GemmArgs& g, int tile, int nN, const char** x,
                                          const char** w) {
    const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
    const long long K = g.K;
    *x = reinterpret_cast<const char*>(static_cast<const T*>(g.A) + m0 * K);
    *w = reinterpret_cast<const char*>(static_cast<const T*>(g.Bt) +
                                       (long long)(m0 / g.rows_per_batch) * g.bt_batch_stride + n0 * K);
}

// Scheduling-group masks (LLVM AMDGPU IGroupLP): MFMA and LDS-read instructions.
constexpr int kSchedMfma = 0x008, kSchedDsRead = 0x100;

// One slab step: slab kt of the current tile sits in stage S and its fragments in
// `f` (one register set per 32-byte half kk). The MFMAs of half 0 go first; then
// the step waits for slab kt+1 and meets the other waves (after which stage S is
// free), issues the 8 direct loads of slab kt+4 into stage S, and reads slab
// kt+1's half-0 fragments into the half-0 registers while the half-1 MFMAs run,
// then its half-1 fragments (consumed in the next step's second half). The
// matrix cores keep working through the barrier and nothing waits for LDS inside
// the step. The last step of a tile reads nothing: slab 0 of the next tile is
// read after the epilogue. Past the last slab of the last tile the loads refetch
// a valid slab, so every step issues the same loads and the vmcnt bookkeeping
// stays uniform.
template <typename T, int S, bool kFirstSlab, bool kReadNext>
__device__ __forceinline__ void slab_step(const Walk& wk, int kt, int wave, unsigned char* lds,
                                          const FragBase& fb, f32x16 (&acc)[4][4], Frags& f,
                                          int younger) {
    constexpr int kPer = sizeof(T) == 2 ? 1 : 4;  // MFMA instructions per group
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, 16>([&](auto m) {
        constexpr int M = decltype(m)::value;
        mfma_group<T, kFirstSlab, M>(acc, f);
    });
    wait_vm(younger);
    lds_barrier();  // slab kt+1 is in LDS; every wave is done reading stage S
    const int ks = kt + 4;
    const bool same = ks < wk.nk;
    issue_slab(same ? wk.x_cur : wk.x_nxt, same ? wk.w_cur : wk.w_nxt, wk.row_bytes,
               same ? ks : ks - wk.nk, wave, wk.voff, lds_addr(lds + S * kStageB));
    const unsigned char* rd = lds + ((S + 1) & 3) * kStageB;
    if constexpr (kReadNext)
        static_for<0, 8>([&](auto r) { read_frag<decltype(r)::value>(f, rd, fb); });
    static_for<16, 32>([&](auto m) {
        constexpr int M = decltype(m)::value;
        mfma_group<T, false, M>(acc, f);
    });
    if constexpr (kReadNext) {
        static_for<8, 16>([&](auto r) { read_frag<decltype(r)::value>(f, rd, fb); });
        static_for<0, 8>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * kPer, 0);
        });
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Four slab steps kb..kb+3 (stages 0..3). kFirst: the tile's first group (zero
// start, and after an epilogue the stores count as younger than slabs 1..3);
// kLast: the tile's last group (its last step reads no next fragments).
template <typename T, bool kFirst, bool kLast>
__device__ __forceinline__ void slab_group(const Walk& wk, int kb, int wave, unsigned char* lds,
                                           const FragBase& fb, f32x16 (&acc)[4][4], Frags& f,
                                           int y_first) {
    constexpr int y = 2 * kDmaPerSlab;
    slab_step<T, 0, kFirst, true>(wk, kb + 0, wave, lds, fb, acc, f, kFirst ? y_first : y);
    slab_step<T, 1, false, true>(wk, kb + 1, wave, lds, fb, acc, f, kFirst ? y_first : y);
    slab_step<T, 2, false, true>(wk, kb + 2, wave, lds, fb, acc, f, kFirst ? y_first : y);
    slab_step<T, 3, false, !kLast>(wk, kb + 3, wave, lds, fb, acc, f, y);
}

// ---- bf16 epilogue ------------------------------------------------------------------
// The tile is first converted (activation, bf16) into registers, 4 consecutive
// channels per piece; it then leaves through a per-wave LDS staging region one
// group (32 rows x 64 columns) at a time -- written in the MFMA layout, read back
// row-contiguous -- so each store writes eight whole 128-byte row segments. Two
// groups are in flight: group g+1 is staged while group g's read-back lands.
struct OutBuf {
    uint2 v[8][8];  // [group 2j + p][4 ii + q]: 4 consecutive channels, bf16
};

template <int kAct>
__device__ __forceinline__ void convert_tile(f32x16 (&acc)[4][4], OutBuf& ob) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            pin_acc(acc[2 * p][j]);
            pin_acc(acc[2 * p + 1][j]);
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = 2 * p + ii;
                    ob.v[2 * j + p][4 * ii + q] = make_uint2(
                        pack_bf16x2(act_of<kAct>(acc[i][j][4 * q + 0]), act_of<kAct>(acc[i][j][4 * q + 1])),
                        pack_bf16x2(act_of<kAct>(acc[i][j][4 * q + 2]), act_of<kAct>(acc[i][j][4 * q + 3])));
                }
        }
}

// Staging of one group: lane (row r32 = lane % 32, half = lane / 32) writes its 8
// pieces of 4 channels; read back, lane l takes 16 bytes of row l/8 (+8 s4).
template <int Gr>
__device__ __forceinline__ void stage_write(const OutBuf& ob, unsigned char* wp) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint2*>(wp + (ii * 32 + 8 * q) * 2) = ob.v[Gr][4 * ii + q];
}
__device__ __forceinline__ void stage_read(const unsigned char* rp, uint4 (&tmp)[4]) {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) tmp[s4] = *reinterpret_cast<const uint4*>(rp + s4 * 8 * kEpiRowB);
}
template <int Gr>
__device__ __forceinline__ void store_group(char* ob, unsigned gl, int ncol, const uint4 (&tmp)[4]) {
    constexpr int j = Gr >> 1, p = Gr & 1;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        const long long uoff = ((long long)(j * 32 + s4 * 8) * ncol + p * 64) * 2;  // uniform
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, tmp[s4]),
                                    reinterpret_cast<u32x4*>(ob + uoff + gl));
    }
}

template <int kAct>
__device__ __forceinline__ void store_tile_bf16(f32x16 (&acc)[4][4], char* ob, int ncol,
                                                unsigned char* ep_w, const unsigned char* ep_r,
                                                unsigned gl) {
    OutBuf obuf;
    convert_tile<kAct>(acc, obuf);
    uint4 t[2][4];
    stage_write<0>(obuf, ep_w);
    stage_read(ep_r, t[0]);
    static_for<1, 8>([&](auto gc) {
        constexpr int Gr = decltype(gc)::value;
        stage_write<Gr>(obuf, ep_w);  // LDS keeps each wave's order: after read Gr-1
        stage_read(ep_r, t[Gr & 1]);
        store_group<Gr - 1>(ob, gl, ncol, t[(Gr - 1) & 1]);
    });
    store_group<7>(ob, gl, ncol, t[1]);
}

template <typename T>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[4 * kStageB];
    constexpr bool kBf16 = sizeof(T) == 2;
    // bf16 epilogue staging, one region per wave (the stages hold the next tile's
    // first slabs while the epilogue runs).
    __shared__ __attribute__((aligned(16))) unsigned char epi[kBf16 ? 4 * kEpiWaveB : 16];
    constexpr int kStores = kBf16 ? kStoresBf16 : kStoresF32;
    constexpr int kSlabE = kSlabB / (int)sizeof(T);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS addresses
    const int wm = wave & 1, wn = wave >> 1;
    const int r32 = lane & 31, half = lane >> 5;

    Walk wk;
    wk.nN = g.N / kBN;
    wk.nk = g.K / kSlabE;  // slabs per tile, a multiple of 4
    wk.row_bytes = (long long)g.K * (long long)sizeof(T);
    // Direct loads: lane l fills physical chunk l%4 of row l/4 of a 16-row group whose
    // first row is a multiple of 32 for even waves and 16 more for odd ones.
    const int dma_row = lane >> 2;
    const int dma_chunk = (lane & 3) ^ row_swz(16 * (wave & 1) + dma_row);
    wk.voff = (unsigned)(dma_row * wk.row_bytes + dma_chunk * 16);
    const int ntiles = (g.M / kBM) * wk.nN;
    if ((gridDim.x & 7) == 0) {
        const int per_xcd_wg = gridDim.x >> 3;
        const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
        const int span = (ntiles + 7) >> 3;
        const int begin = xcd * span;
        wk.tile_end = min(ntiles, begin + span);
        wk.tile = begin + j;
        wk.stride = per_xcd_wg;
    } else {
        wk.tile = blockIdx.x;
        wk.stride = gridDim.x;
        wk.tile_end = ntiles;
    }
    if (wk.tile >= wk.tile_end) return;

    FragBase fbase;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        const unsigned lane_part = r32 * kSlabB + (((2 * kk + half) ^ row_swz(r32)) << 4);
        fbase.x[kk] = lane_part + (wm * 128) * kSlabB;
        fbase.w[kk] = lane_part + (kBM + wn * 128) * kSlabB;
    }

    // Prologue: slabs 0..3 of the first tile, then slab 0's fragments.
    tile_rows<T>(g, wk.tile, wk.nN, &wk.x_cur, &wk.w_cur);
#pragma unroll
    for (int s = 0; s < 4; ++s)
        issue_slab(wk.x_cur, wk.w_cur, wk.row_bytes, s, wave, wk.voff, lds_addr(lds + s * kStageB));
    wait_vm(3 * kDmaPerSlab);
    lds_barrier();
    Frags fa;
    static_for<0, 16>([&](auto r) { read_frag<decltype(r)::value>(fa, lds, fbase); });

    bool stores_pending = false;  // the previous tile's stores follow slabs 0..3 of this one
    f32x16 acc[4][4];
    unsigned char* ep_w = epi + wave * kEpiWaveB + r32 * kEpiRowB + half * 8;
    const unsigned char* ep_r = epi + wave * kEpiWaveB + (lane >> 3) * kEpiRowB + (lane & 7) * 16;
    const unsigned ep_gl = (unsigned)(((lane >> 3) * g.ncol + (lane & 7) * 8) * 2);
    while (true) {
        wk.next = wk.tile + wk.stride < wk.tile_end ? wk.tile + wk.stride : -1;
        if (wk.next >= 0) tile_rows<T>(g, wk.next, wk.nN, &wk.x_nxt, &wk.w_nxt);
        else wk.x_nxt = wk.x_cur, wk.w_nxt = wk.w_cur;
        // Loads younger than slab kt+1 when step kt waits for it: slabs kt+2 and
        // kt+3, and for kt <= 2 after an epilogue also that epilogue's stores.
        constexpr int y_store = kStores + 2 * kDmaPerSlab <= 63 ? kStores + 2 * kDmaPerSlab : 0;
        const int y_first = stores_pending ? y_store : 2 * kDmaPerSlab;
        if (wk.nk == 4) {
            slab_group<T, true, true>(wk, 0, wave, lds, fbase, acc, fa, y_first);
        } else {
            slab_group<T, true, false>(wk, 0, wave, lds, fbase, acc, fa, y_first);
            for (int kb = 4; kb < wk.nk - 4; kb += 4)
                slab_group<T, false, false>(wk, kb, wave, lds, fbase, acc, fa, 0);
            slab_group<T, false, true>(wk, wk.nk - 4, wave, lds, fbase, acc, fa, 0);
        }
        // Slab 0 of the next tile is in stage 0 (published by the last step's barrier);
        // its fragments are read after the epilogue.
        const int m0 = (wk.tile / wk.nN) * kBM, n0 = (wk.tile % wk.nN) * kBN;
        const int plane = n0 / g.ncol;
        T* out = static_cast<T*>(g.out[plane]);
        const int col0 = n0 - plane * g.ncol + wn * 128;
        // The whole 256-wide N tile lies in one output plane: uniform activation.
        if constexpr (kBf16) {
            char* obase = reinterpret_cast<char*>(reinterpret_cast<bf16_t*>(out) +
                                                  (long long)(m0 + wm * 128) * g.ncol + col0);
            // The distinct markers keep the compiler from hoisting the accumulator
            // reads common to the three arms above the switch (all 256 at once).
            switch (g.act[plane]) {
                case 1:
                    asm volatile("; epilogue relu");
                    store_tile_bf16<1>(acc, obase, g.ncol, ep_w, ep_r, ep_gl);
                    break;
                case 2:
                    asm volatile("; epilogue gelu");
                    store_tile_bf16<2>(acc, obase, g.ncol, ep_w, ep_r, ep_gl);
                    break;
                default:
                    asm volatile("; epilogue identity");
                    store_tile_bf16<0>(acc, obase, g.ncol, ep_w, ep_r, ep_gl);
                    break;
            }
        } else {
            float* obase = reinterpret_cast<float*>(out) + (long long)(m0 + wm * 128 + r32) * g.ncol +
                           col0 + 4 * half;
            switch (g.act[plane]) {
                case 1:
                    asm volatile("; epilogue relu");
                    store_tile_f32<1>(acc, obase, g.ncol);
                    break;
                case 2:
                    asm volatile("; epilogue gelu");
                    store_tile_f32<2>(acc, obase, g.ncol);
                    break;
                default:
                    asm volatile("; epilogue identity");
                    store_tile_f32<0>(acc, obase, g.ncol);
                    break;
            }
        }
        stores_pending = true;
        if (wk.next < 0) break;
        static_for<0, 16>([&](auto r) { read_frag<decltype(r)::value>(fa, lds, fbase); });
        wk.tile = wk.next;
        wk.x_cur = wk.x_nxt;
        wk.w_cur = wk.w_nxt;
    }
    // Loads refetched past the last slab may still be landing in LDS.
    wait_vm(0);
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
        const float s = scaled ? w.scale[b * heads + head] : 1.0f;
        if constexpr (sizeof(T) == 2) {
            *reinterpret_cast<uint4*>(static_cast<T*>(w.Wt) + (long long)b * per_b + r) =
                make_uint4(pack_bf16x2(v0.x * s, v0.y * s), pack_bf16x2(v0.z * s, v0.w * s),
                           pack_bf16x2(v1.x * s, v1.y * s), pack_bf16x2(v1.z * s, v1.w * s));
        } else {
            float* dst = static_cast<float*>(w.Wt) + (long long)b * per_b + r;
            *reinterpret_cast<float4*>(dst) = make_float4(v0.x * s, v0.y * s, v0.z * s, v0.w * s);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(v1.x * s, v1.y * s, v1.z * s, v1.w * s);
        }
    }
}
}  // namespace

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
