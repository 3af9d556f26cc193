// gemm_tile.hpp — the MFMA tile kernel of the [P|I|V] projections (gemm.hip), kept in
// a header so that other translation units can build its backward variants:
// gemm_add.hip with SLIME_GEMM_ADD (one fp32 output plane written as the product plus
// an addend: dL/dX = the direct part + the part through the projections) and
// gemm_tape.hip with SLIME_GEMM_TAPE (the forward projections, the GELU plane also
// written before its activation, for the backward's tape). Without either macro this
// is exactly the forward kernel.
#pragma once

#include <type_traits>

#include "common.hpp"
#include "gemm_addr.hpp"
#include "kernels.hpp"

namespace slime {
namespace {

// Tile shape, ring and staging constants, and all address arithmetic: gemm_addr.hpp.
// Stage layout: tile row r (0..255 cells, 256..511 output channels) holds its 64
// slab bytes at r*64, as four 16-byte chunks XOR-permuted by
// f(r) = row_swz(r) = (r >> 2) & 3: physical chunk = logical chunk ^ f(r). One
// direct-load instruction fills 16 whole rows (1 KiB, four lanes per 64-byte row),
// and the operand reads -- 32 consecutive rows at one logical chunk per half
// wave -- fall in distinct LDS bank groups in every pass (gemm_addr.hpp).
using namespace gemm_addr;

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
#pragma unroll
        for (int i = 0; i < 4; ++i) pin_acc(acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4*>(obase + f32_store_elem(j, i, q, ncol)) =
                    make_float4(act_of<kAct>(acc[i][j][4 * q + 0]), act_of<kAct>(acc[i][j][4 * q + 1]),
                                act_of<kAct>(acc[i][j][4 * q + 2]), act_of<kAct>(acc[i][j][4 * q + 3]));
    }
}

#ifdef SLIME_GEMM_ADD
// fp32 epilogue with an addend of the output's layout: out = acc + add (in place
// allowed: each element is read and written by the same lane).
__device__ __forceinline__ void store_tile_f32_add(f32x16 (&acc)[4][4], float* obase, const float* abase,
                                                   int ncol) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float4 ad[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) ad[i][q] = *reinterpret_cast<const float4*>(abase + f32_store_elem(j, i, q, ncol));
#pragma unroll
        for (int i = 0; i < 4; ++i) pin_acc(acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4*>(obase + f32_store_elem(j, i, q, ncol)) =
                    make_float4(acc[i][j][4 * q + 0] + ad[i][q].x, acc[i][j][4 * q + 1] + ad[i][q].y,
                                acc[i][j][4 * q + 2] + ad[i][q].z, acc[i][j][4 * q + 3] + ad[i][q].w);
    }
}
#endif

// Direct global->LDS loads: dma16_lds (common.hpp). The pipeline waits for each slab
// itself (wait_vm) before the barrier that publishes it.

// Issues the direct global->LDS loads of slab ks of a tile into the stage at LDS
// byte address sbase: 32 instructions of 16 rows each; wave w issues row groups
// w, w+4, ..., w+28 (16 cell groups, then 16 weight groups). x, w: the tile's
// first cell row and first weight row (uniform); voff: this lane's byte offset
// (row lane/4 of the group, the logical chunk that lands in physical chunk lane%4).
__device__ __forceinline__ void issue_slab(const char* x, const char* w, long long row_bytes, int ks,
                                           int wave, unsigned voff, unsigned sbase) {
    const long long k_off = dma_k_off(ks);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16_lds(x + dma_grp_off(j, wave, row_bytes) + k_off, voff, sbase + dma_lds_off(j, wave));
#pragma unroll
    for (int j = 4; j < 8; ++j) dma16_lds(w + dma_grp_off(j, wave, row_bytes) + k_off, voff, sbase + dma_lds_off(j, wave));
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
        f.x[kk][q] = *reinterpret_cast<const u32x4*>(stage + b.x[kk] + frag_block_off(q));
    else
        f.w[kk][q - 4] = *reinterpret_cast<const u32x4*>(stage + b.w[kk] + frag_block_off(q - 4));
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
    long long xe, we;
    tile_row_elems(tile, nN, g.K, g.rows_per_batch, g.bt_batch_stride, &xe, &we);
    *x = reinterpret_cast<const char*>(static_cast<const T*>(g.A) + xe);
    *w = reinterpret_cast<const char*>(static_cast<const T*>(g.Bt) + we);
}


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
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, 16>([&](auto m) {
        constexpr int M = decltype(m)::value;
        mfma_group<T, kFirstSlab, M>(acc, f);
    });
    wait_vm(younger);
    lds_barrier();  // slab kt+1 is in LDS; every wave is done reading stage S
    const int ks = kt + 4;
    const bool same = ks < wk.nk;
    // The half-1 MFMAs go out in pairs, each pair after one direct load of slab kt+4
    // and one fragment read of slab kt+1: when the memory pipeline is backed up and
    // a load waits to issue, the matrix core still has the previous pair queued.
    const char* xs = same ? wk.x_cur : wk.x_nxt;
    const char* ws = same ? wk.w_cur : wk.w_nxt;
    const long long k_off = dma_k_off(same ? ks : ks - wk.nk);
    const unsigned sb = lds_addr(lds + S * kStageB);
    const unsigned char* rd = lds + ((S + 1) & 3) * kStageB;
    static_for<0, kDmaPerSlab>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        __builtin_amdgcn_sched_barrier(0);
        dma16_lds((j < 4 ? xs : ws) + dma_grp_off(j, wave, wk.row_bytes) + k_off, wk.voff, sb + dma_lds_off(j, wave));
        if constexpr (kReadNext) read_frag<j>(f, rd, fb);
        mfma_group<T, false, 16 + 2 * j>(acc, f);
        mfma_group<T, false, 17 + 2 * j>(acc, f);
        __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (kReadNext) static_for<8, 16>([&](auto r) { read_frag<decltype(r)::value>(f, rd, fb); });
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
            for (int ii = 0; ii < 2; ++ii) {
                const int i = 2 * p + ii;
                if constexpr (kAct == 2) {
                    // GELU of the block's 16 values stage by stage: their exp2 and rcp
                    // issue back to back instead of one value's chain at a time.
                    float v[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e];
                    gelu_tanh_n(v);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        ob.v[2 * j + p][4 * ii + q] = make_uint2(pack_bf16x2(v[4 * q + 0], v[4 * q + 1]),
                                                                 pack_bf16x2(v[4 * q + 2], v[4 * q + 3]));
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        ob.v[2 * j + p][4 * ii + q] = make_uint2(
                            pack_bf16x2(act_of<kAct>(acc[i][j][4 * q + 0]), act_of<kAct>(acc[i][j][4 * q + 1])),
                            pack_bf16x2(act_of<kAct>(acc[i][j][4 * q + 2]), act_of<kAct>(acc[i][j][4 * q + 3])));
                }
            }
        }
}

// Staging of one group: lane (row r32 = lane % 32, half = lane / 32) writes its 8
// pieces of 4 channels; read back, lane l takes 16 bytes of row l/8 (+8 s4). The
// staging layout (gemm_addr.hpp) is free of bank conflicts; rows with bit 3 set hold
// their chunk halves swapped, undone here in registers.
template <int Gr>
__device__ __forceinline__ void stage_write(const OutBuf& ob, unsigned char* epi, unsigned w_off) {
#pragma unroll
    for (int k = 0; k < 8; ++k) *reinterpret_cast<uint2*>(epi + epi_w_piece(w_off, k)) = ob.v[Gr][k];
}
__device__ __forceinline__ void stage_read(const unsigned char* rp, uint4 (&tmp)[4]) {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        const uint4 v = *reinterpret_cast<const uint4*>(rp + s4 * 8 * kEpiRowB);
        tmp[s4] = epi_r_swapped(s4) ? make_uint4(v.z, v.w, v.x, v.y) : v;
    }
}
template <int Gr>
__device__ __forceinline__ void store_group(char* ob, unsigned gl, int ncol, const uint4 (&tmp)[4]) {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        const long long uoff = bf16_store_off(Gr, s4, ncol);  // uniform
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, tmp[s4]),
                                    reinterpret_cast<u32x4*>(ob + uoff + gl));
    }
}

template <int kAct>
__device__ __forceinline__ void store_tile_bf16(f32x16 (&acc)[4][4], char* ob, int ncol,
                                                unsigned char* epi, unsigned ep_w, const unsigned char* ep_r,
                                                unsigned gl) {
    OutBuf obuf;
    convert_tile<kAct>(acc, obuf);
    uint4 t[2][4];
    stage_write<0>(obuf, epi, ep_w);
    stage_read(ep_r, t[0]);
    static_for<1, 8>([&](auto gc) {
        constexpr int Gr = decltype(gc)::value;
        stage_write<Gr>(obuf, epi, ep_w);  // LDS keeps each wave's order: after read Gr-1
        stage_read(ep_r, t[Gr & 1]);
        store_group<Gr - 1>(ob, gl, ncol, t[(Gr - 1) & 1]);
    });
    store_group<7>(ob, gl, ncol, t[1]);
}

#ifdef SLIME_GEMM_TAPE
// The identity epilogue of a tile whose accumulators stay live afterwards (the tape
// kernel's pre-activation plane): each group (32 rows x 64 columns: accumulator
// blocks [2p][j] and [2p+1][j] of group 2j+p) is converted just before it is staged,
// so one group's bf16 values are held at a time rather than the whole tile's, and
// the pass needs no registers the accumulators would otherwise free. The stores are
// those of store_tile_bf16<0>: same bytes, same places.
template <int Gr>
__device__ __forceinline__ void convert_group_identity(f32x16 (&acc)[4][4], uint2 (&v)[8]) {
    constexpr int j = Gr / 2, p = Gr % 2;
    pin_acc(acc[2 * p][j]);
    pin_acc(acc[2 * p + 1][j]);
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            v[4 * ii + q] = make_uint2(pack_bf16x2(acc[2 * p + ii][j][4 * q + 0], acc[2 * p + ii][j][4 * q + 1]),
                                       pack_bf16x2(acc[2 * p + ii][j][4 * q + 2], acc[2 * p + ii][j][4 * q + 3]));
}
__device__ __forceinline__ void stage_write_group(const uint2 (&v)[8], unsigned char* epi, unsigned w_off) {
#pragma unroll
    for (int k = 0; k < 8; ++k) *reinterpret_cast<uint2*>(epi + epi_w_piece(w_off, k)) = v[k];
}
__device__ __forceinline__ void store_tile_bf16_identity_lean(f32x16 (&acc)[4][4], char* ob, int ncol,
                                                              unsigned char* epi, unsigned ep_w,
                                                              const unsigned char* ep_r, unsigned gl) {
    uint2 v[2][8];
    uint4 t[2][4];
    convert_group_identity<0>(acc, v[0]);
    stage_write_group(v[0], epi, ep_w);
    stage_read(ep_r, t[0]);
    static_for<1, 8>([&](auto gc) {
        constexpr int Gr = decltype(gc)::value;
        convert_group_identity<Gr>(acc, v[Gr & 1]);
        stage_write_group(v[Gr & 1], epi, ep_w);
        stage_read(ep_r, t[Gr & 1]);
        store_group<Gr - 1>(ob, gl, ncol, t[(Gr - 1) & 1]);
    });
    store_group<7>(ob, gl, ncol, t[1]);
}
#endif

template <typename T>
#if defined(SLIME_GEMM_ADD)
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_add_kernel(GemmArgs g, const float* add) {
#elif defined(SLIME_GEMM_TAPE)
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_tape_kernel(GemmArgs g, void* pre) {
#else
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(GemmArgs g) {
#endif
    __shared__ __attribute__((aligned(1024))) unsigned char lds[4 * kStageB];
    constexpr bool kBf16 = sizeof(T) == 2;
    // bf16 epilogue staging, one region per wave (the stages hold the next tile's
    // first slabs while the epilogue runs).
    __shared__ __attribute__((aligned(128))) unsigned char epi[kBf16 ? 4 * kEpiWaveB : 16];
#ifndef SLIME_GEMM_ADD
    constexpr int kStores = kBf16 ? kStoresBf16 : kStoresF32;
#else
    constexpr int kStores = kStoresF32;
#endif
    constexpr int kSlabE = kSlabB / (int)sizeof(T);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS addresses

    Walk wk;
    wk.nN = g.N / kBN;
    wk.nk = g.K / kSlabE;  // slabs per tile, a multiple of 4
    wk.row_bytes = (long long)g.K * (long long)sizeof(T);
    wk.voff = dma_lane_off(wave, lane, wk.row_bytes);
    const int ntiles = (g.M / kBM) * wk.nN;
    const Sched sc = schedule(blockIdx.x, gridDim.x, ntiles);
    wk.tile = sc.tile;
    wk.stride = sc.stride;
    wk.tile_end = sc.tile_end;
    if (wk.tile >= wk.tile_end) return;

    FragBase fbase;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        fbase.x[kk] = frag_x_off(kk, lane, wave);
        fbase.w[kk] = frag_w_off(kk, lane, wave);
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
    const unsigned ep_w = epi_w_off(wave, lane);
    const unsigned char* ep_r = epi + epi_r_off(wave, lane);
    const unsigned ep_gl = epi_gl_off(lane, g.ncol);
    while (true) {
        wk.next = wk.tile + wk.stride < wk.tile_end ? wk.tile + wk.stride : -1;
        if (wk.next >= 0) tile_rows<T>(g, wk.next, wk.nN, &wk.x_nxt, &wk.w_nxt);
        else wk.x_nxt = wk.x_cur, wk.w_nxt = wk.w_cur;
        // Loads younger than slab kt+1 when step kt waits for it: slabs kt+2 and
        // kt+3, and for kt <= 2 after an epilogue also that epilogue's stores (after
        // the tape variant's two epilogues of a GELU tile, more than are counted:
        // the wait then also covers some of those stores).
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
        const int plane = tile_plane(wk.tile, wk.nN, g.ncol);
        T* out = static_cast<T*>(g.out[plane]);
        const long long wave_el = wave_out_elem(wk.tile, wk.nN, g.ncol, wave);
        // The whole 256-wide N tile lies in one output plane: uniform activation.
#ifdef SLIME_GEMM_ADD
        if constexpr (true) {
            const long long off = wave_el + f32_lane_elem(lane, g.ncol);
            store_tile_f32_add(acc, static_cast<float*>(g.out[plane]) + off, add + off, g.ncol);
        } else
#endif
#ifdef SLIME_GEMM_TAPE
        if (g.act[plane] == 2) {  // the GELU plane also leaves before its activation
            asm volatile("; epilogue pre-activation");
            if constexpr (kBf16)
                store_tile_bf16_identity_lean(acc, reinterpret_cast<char*>(reinterpret_cast<bf16_t*>(pre) + wave_el),
                                              g.ncol, epi, ep_w, ep_r, ep_gl);
            else
                store_tile_f32<0>(acc, static_cast<float*>(pre) + wave_el + f32_lane_elem(lane, g.ncol), g.ncol);
            // Ordered after every store above (memory clobber) and before the second
            // epilogue's accumulator pins (volatile): the two conversions do not
            // overlap, so each holds the registers of one.
            asm volatile("; epilogue pre-activation done" ::: "memory");
        }
#endif
        if constexpr (kBf16) {
            char* obase = reinterpret_cast<char*>(reinterpret_cast<bf16_t*>(out) + wave_el);
            // The distinct markers keep the compiler from hoisting the accumulator
            // reads common to the three arms above the switch (all 256 at once).
            switch (g.act[plane]) {
                case 1:
                    asm volatile("; epilogue relu");
                    store_tile_bf16<1>(acc, obase, g.ncol, epi, ep_w, ep_r, ep_gl);
                    break;
                case 2:
                    asm volatile("; epilogue gelu");
                    store_tile_bf16<2>(acc, obase, g.ncol, epi, ep_w, ep_r, ep_gl);
                    break;
                default:
                    asm volatile("; epilogue identity");
                    store_tile_bf16<0>(acc, obase, g.ncol, epi, ep_w, ep_r, ep_gl);
                    break;
            }
        } else {
            float* obase = reinterpret_cast<float*>(out) + wave_el + f32_lane_elem(lane, g.ncol);
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


}  // namespace
}  // namespace slime
