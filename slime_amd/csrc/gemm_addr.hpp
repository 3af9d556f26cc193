// gemm_addr.hpp — the address arithmetic of the projection GEMM's tile kernel
// (gemm_tile.hpp): the persistent tile schedule, every lane's direct-load source
// offset and LDS destination, the operand fragment reads, and the epilogue's LDS
// staging and global store offsets. Plain C++ with no HIP types, so the kernel and
// a host program share one definition: tests/gemm_addr_replay.cpp replays every
// address of a launch on the host and checks it against the bounds of its buffer,
// and checks the kernel's vmcnt waits against the order its loads and stores issue.
#pragma once

#if defined(__HIPCC__)
#define SLIME_HD __host__ __device__ __forceinline__
#else
#define SLIME_HD inline
#endif

namespace slime {
namespace gemm_addr {

constexpr int kBM = 256, kBN = 256, kThreads = 256, kWaves = kThreads / 64;
constexpr int kSlabB = 64;                     // bytes of K per tile row per slab
constexpr int kStages = 4;                     // LDS ring depth (slabs)
constexpr int kStageB = (kBM + kBN) * kSlabB;  // 32 KiB
constexpr int kDmaPerSlab = 8;                 // direct-load instructions per wave per slab
constexpr int kEpiRowB = 128;                  // bf16 epilogue staging row pitch (no padding)
constexpr int kEpiWaveB = 32 * kEpiRowB;       // staging bytes per wave
constexpr int kStoresBf16 = 32;                // global stores per wave per tile (bf16 epilogue)
constexpr int kStoresF32 = 64;                 // global stores per wave per tile (fp32 epilogue)

// Stage layout: tile row r (0..255 cells, 256..511 output channels) holds its 64
// slab bytes at r*64 as four 16-byte chunks, physical chunk = logical chunk ^ f(r),
// f(r) = (r >> 2) & 3. gfx950 serves a 16-byte LDS read of a wave in four passes of
// 16 lanes -- the lanes 4q..4q+3 of the quads q that share q >> 3 and the parity of
// q & 7 -- over 16 bank groups of 16 bytes (address / 16 % 16), measured with the
// bank-conflict counter. With this f the 16 lanes of every pass of a fragment read
// (row lane % 32 of a block, logical chunk 2 kk + lane / 32) fall in 16 distinct
// groups: no conflict cycles.
SLIME_HD constexpr int row_swz(int r) { return (r >> 2) & 3; }

// One persistent workgroup per CU, never more than there are tiles.
SLIME_HD int grid_size(int ntiles, int n_cu) { return ntiles < n_cu ? ntiles : n_cu; }

// The tiles a workgroup walks: tile, tile + stride, ... below tile_end. With a grid
// that is a multiple of the 8 XCDs (workgroup w runs on XCD w % 8), each XCD walks
// one contiguous eighth of the tiles, so neighbouring tiles share its L2.
struct Sched {
    int tile, stride, tile_end;
};
SLIME_HD Sched schedule(int block, int grid, int ntiles) {
    Sched s;
    if ((grid & 7) == 0) {
        const int per_xcd_wg = grid >> 3;
        const int xcd = block & 7, j = block >> 3;
        const int span = (ntiles + 7) >> 3;
        const int begin = xcd * span;
        s.tile_end = begin + span < ntiles ? begin + span : ntiles;
        s.tile = begin + j;
        s.stride = per_xcd_wg;
    } else {
        s.tile = block;
        s.stride = grid;
        s.tile_end = ntiles;
    }
    return s;
}

// Element offsets of a tile's first cell row in A and first weight row in Bt.
SLIME_HD void tile_row_elems(int tile, int nN, long long K, int rows_per_batch, long long bt_batch_stride,
                             long long* x_el, long long* w_el) {
    const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
    *x_el = m0 * K;
    *w_el = (long long)(m0 / rows_per_batch) * bt_batch_stride + n0 * K;
}

// Direct loads: one instruction fills 16 whole rows (1 KiB), lane l the physical
// chunk l % 4 of row l / 4; this is the lane's byte offset from the group's first
// row (a multiple of 32 rows for even waves, 16 more for odd ones).
SLIME_HD unsigned dma_lane_off(int wave, int lane, long long row_bytes) {
    const int dma_row = lane >> 2;
    const int dma_chunk = (lane & 3) ^ row_swz(16 * (wave & 1) + dma_row);
    return (unsigned)(dma_row * row_bytes + dma_chunk * 16);
}

// Direct load j (0..7) of slab ks by wave `wave`: row group 4 (j % 4) + wave of the
// cells (j < 4) or of the weights (j >= 4). Source: byte offset from the tile's
// first row of that operand; destination: byte offset in the stage (16 bytes per
// lane from there).
SLIME_HD long long dma_grp_off(int j, int wave, long long row_bytes) {
    const int grp = 4 * (j & 3) + wave;
    return grp * 16 * row_bytes;
}
SLIME_HD long long dma_k_off(int ks) { return (long long)ks * kSlabB; }
SLIME_HD long long dma_src_off(int j, int wave, long long row_bytes, int ks) {
    return dma_grp_off(j, wave, row_bytes) + dma_k_off(ks);
}
SLIME_HD unsigned dma_lds_off(int j, int wave) {
    const int grp = 4 * (j & 3) + wave;
    return (unsigned)((j < 4 ? grp : 16 + grp) * 1024);
}

// Operand fragment reads (16 bytes per lane) inside a stage, per 32-byte half kk:
// the wave's first cell row block and first weight row block at row lane % 32 of
// the block, physical chunk of logical chunk 2 kk + lane / 32; block q (0..3) of
// either operand is 32 rows further.
SLIME_HD unsigned frag_x_off(int kk, int lane, int wave) {
    const int r32 = lane & 31, half = lane >> 5, wm = wave & 1;
    return (unsigned)(r32 * kSlabB + (((2 * kk + half) ^ row_swz(r32)) << 4) + (wm * 128) * kSlabB);
}
SLIME_HD unsigned frag_w_off(int kk, int lane, int wave) {
    const int r32 = lane & 31, half = lane >> 5, wn = wave >> 1;
    return (unsigned)(r32 * kSlabB + (((2 * kk + half) ^ row_swz(r32)) << 4) + (kBM + wn * 128) * kSlabB);
}
SLIME_HD unsigned frag_block_off(int q) { return (unsigned)(q * 32 * kSlabB); }

// bf16 epilogue staging in the per-wave region (32 rows of 64 channels, 128 bytes).
// Row r keeps its eight 16-byte chunks (8 channels each) at physical chunk = logical
// chunk ^ (r & 7), and the two 8-byte halves of a chunk (4 channels each) swapped when
// bit 3 of r is set. Write: lane (row r = lane % 32, half h = lane / 32) stores its
// 8 bytes of logical chunk k at epi_w_off(wave, lane) ^ (k << 4) (the XOR only touches
// the chunk bits). Read: lane l takes row l / 8 + 8 s4, logical chunk l % 8, at
// epi_r_off(wave, lane) + s4 * 8 * kEpiRowB, halves swapped for odd s4. Every pass of
// the 8-byte writes (16 lanes over 16 groups of 8 bytes) and of the 16-byte reads
// falls in distinct bank groups.
SLIME_HD unsigned epi_w_off(int wave, int lane) {
    const int r = lane & 31, h = lane >> 5;
    return (unsigned)(wave * kEpiWaveB + r * kEpiRowB + ((r & 7) << 4) + ((h ^ ((r >> 3) & 1)) << 3));
}
SLIME_HD unsigned epi_w_piece(unsigned w_off, int k) { return w_off ^ (unsigned)(k << 4); }
SLIME_HD unsigned epi_r_off(int wave, int lane) {
    const int r = lane >> 3;  // row inside each run of 8 rows
    return (unsigned)(wave * kEpiWaveB + r * kEpiRowB + (((lane & 7) ^ r) << 4));
}
SLIME_HD bool epi_r_swapped(int s4) { return (s4 & 1) != 0; }

// Output of a tile: plane n0 / ncol; the wave's first output element in that plane
// (row m0 + 128 wm, column n0 - plane ncol + 128 wn).
SLIME_HD int tile_plane(int tile, int nN, int ncol) { return ((tile % nN) * kBN) / ncol; }
SLIME_HD long long wave_out_elem(int tile, int nN, int ncol, int wave) {
    const int m0 = (tile / nN) * kBM, n0 = (tile % nN) * kBN;
    const int plane = n0 / ncol;
    return (long long)(m0 + (wave & 1) * 128) * ncol + (n0 - plane * ncol + (wave >> 1) * 128);
}
// bf16 epilogue: lane's 16-byte store (group gr < 8, piece s4 < 4) at this byte
// offset from the wave's first output element.
SLIME_HD unsigned epi_gl_off(int lane, int ncol) {
    return (unsigned)(((lane >> 3) * ncol + (lane & 7) * 8) * 2);
}
SLIME_HD long long bf16_store_off(int gr, int s4, int ncol) {
    const int j = gr >> 1, p = gr & 1;
    return ((long long)(j * 32 + s4 * 8) * ncol + p * 64) * 2;
}
// fp32 epilogue: lane's 16-byte store (j, i, q < 4) at this element offset from the
// wave's first output element.
SLIME_HD long long f32_lane_elem(int lane, int ncol) { return (long long)(lane & 31) * ncol + 4 * (lane >> 5); }
SLIME_HD long long f32_store_elem(int j, int i, int q, int ncol) {
    return (long long)j * 32 * ncol + i * 32 + 8 * q;
}

}  // namespace gemm_addr
}  // namespace slime
