// Host replay of every address the projection GEMM's tile kernel (gemm_tile.hpp)
// issues for one launch, through the kernel's own address functions
// (slime_amd/csrc/gemm_addr.hpp). Test infrastructure: built with g++ by
// tests/test_gemm_addr.py; nothing in the library uses it.
//
// For every workgroup of the persistent grid, every wave and every lane it checks:
//   * each direct load's 16-byte source lies inside A or Bt, and its LDS
//     destination inside the 4-stage ring;
//   * each operand fragment read lies inside its stage, reads the slab that the
//     stage holds, and that slab was covered by an earlier wait of this wave;
//   * each vmcnt wait covers the slab it publishes under in-order completion of
//     the wave's vector-memory operations (the direct loads and the epilogue's
//     stores), and is exactly as tight as that (no looser, no stricter);
//   * the bf16 epilogue's LDS staging stays inside the wave's own region;
//   * the LDS layouts carry the data: each fragment read finds the tile row and
//     16-byte chunk its MFMA needs, and each staged read-back the row and channels
//     its global store writes (check_layouts);
//   * each global store (and, for the adding epilogue, each addend load) lies
//     inside its output plane;
//   * the workgroups together visit every tile exactly once.
//
// Usage: gemm_addr_replay M N K elem rows_per_batch bt_batch_stride bt_elems
//                         ncol nplanes n_cu epilogue
//   elem: 2 (bf16) or 4 (fp32) operands; epilogue: bf16 | f32 | f32add
//   optional 12th argument "plant-loose-wait": model every slab wait 8 operations
//   looser than the kernel's (a planted mistake, so tests can see the check fire)
// Prints "OK ..." and exits 0, or prints the first violation and exits 1.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "../slime_amd/csrc/gemm_addr.hpp"

using namespace slime::gemm_addr;

namespace {

struct Launch {
    long long M, N, K, elem, rows_per_batch, bt_batch_stride, bt_elems, ncol, nplanes, n_cu;
    std::string epi;
    int plant = 0;  // added to every modelled slab wait
};

long long g_checks = 0;

[[noreturn]] void fail(const char* what, long long a, long long b, long long c) {
    std::printf("FAIL %s (%lld, %lld, %lld)\n", what, a, b, c);
    std::exit(1);
}

void in_range(const char* what, long long off, long long len, long long size) {
    ++g_checks;
    if (off < 0 || off + len > size) fail(what, off, len, size);
}

// One slab's identity: (tile, k slab); tile -1 = none.
struct SlabId {
    int tile = -1, ks = -1;
    bool operator==(const SlabId& o) const { return tile == o.tile && ks == o.ks; }
};

// A wave's in-order vector-memory operations: the slab each direct load fills
// (stores carry tile -2).
struct Wave {
    std::vector<SlabId> ops;
    SlabId stage[kStages];
    std::vector<SlabId> covered;  // slabs a wait has confirmed complete

    void issue(SlabId s) { ops.push_back(s); }
    // s_waitcnt vmcnt(n) before the barrier that publishes slab `need`.
    long long done = 0;  // ops[0, done) are known complete
    void wait(int n, SlabId need) {
        long long last = -1;
        for (long long i = (long long)ops.size() - 1; i >= 0 && last < 0; --i)
            if (ops[i] == need) last = i;
        if (last < 0) fail("wait for a slab never loaded", need.tile, need.ks, n);
        const long long younger = (long long)ops.size() - 1 - last;
        if (n > 63) fail("vmcnt immediate beyond the 6-bit counter", n, 0, 0);
        if (last >= done) {
            if (n > younger) fail("vmcnt wait too loose: slab may be incomplete", need.ks, n, younger);
            if (n < younger && n != 0) fail("vmcnt wait stricter than needed", need.ks, n, younger);
        }
        // in-order completion: everything but the n youngest has completed
        if ((long long)ops.size() - n > done) done = (long long)ops.size() - n;
        if (covered.size() > 64) covered.erase(covered.begin(), covered.begin() + 32);
        covered.push_back(need);
        ++g_checks;
    }
    void drain() { done = (long long)ops.size(); }
    void read(int st, SlabId want) {
        if (!(stage[st] == want)) fail("fragment read from a stage holding another slab", st, want.ks, stage[st].ks);
        bool ok = false;
        for (const SlabId& c : covered) ok = ok || c == want;
        if (!ok) fail("fragment read of a slab no wait covered", want.tile, want.ks, st);
        ++g_checks;
    }
};

// The data path through the LDS layouts, independent of the tile: every 16-byte slot
// of a stage is filled by exactly one direct-load lane, and each operand fragment read
// finds there the tile row and logical 16-byte chunk of the slab that its MFMA needs;
// every 8-byte slot of a wave's epilogue staging region is written by exactly one
// (lane, piece), and each read-back (with its halves put back in order) holds the row
// and chunk that its global store sends to that row and those channels.
void check_layouts(long long row_bytes, long long ncol) {
    struct Slot { int row = -1, chunk = -1; };
    std::vector<Slot> stage(kStageB / 16);
    for (int wave = 0; wave < kWaves; ++wave)
        for (int j = 0; j < kDmaPerSlab; ++j)
            for (int lane = 0; lane < 64; ++lane) {
                const long long src = dma_grp_off(j, wave, row_bytes) + dma_lane_off(wave, lane, row_bytes);
                const long long b = dma_lds_off(j, wave) + 16LL * lane;
                in_range("direct-load destination inside the stage", b, 16, kStageB);
                Slot& sl = stage[b / 16];
                if (sl.row >= 0) fail("stage slot filled twice", b, wave, lane);
                sl.row = (int)(src / row_bytes) + (j < 4 ? 0 : kBM);
                sl.chunk = (int)((src % row_bytes) / 16);
                if (src % 16 || sl.chunk >= kSlabB / 16) fail("direct-load source off a 16-byte chunk of the slab", src, wave, lane);
            }
    for (size_t i = 0; i < stage.size(); ++i)
        if (stage[i].row < 0) fail("stage slot never filled", (long long)i, 0, 0);
    for (int wave = 0; wave < kWaves; ++wave)
        for (int lane = 0; lane < 64; ++lane)
            for (int kk = 0; kk < 2; ++kk)
                for (int q = 0; q < 4; ++q) {
                    const int r32 = lane & 31, chunk = 2 * kk + (lane >> 5);
#ifdef PLANT_FRAG_CHUNK  // a planted mistake: the cell fragment reads its chunk's neighbour
                    const Slot& x = stage[((frag_x_off(kk, lane, wave) ^ 16u) + frag_block_off(q)) / 16];
#else
                    const Slot& x = stage[(frag_x_off(kk, lane, wave) + frag_block_off(q)) / 16];
#endif
                    if (x.row != r32 + 32 * q + 128 * (wave & 1) || x.chunk != chunk)
                        fail("cell fragment reads the wrong row or chunk", lane, kk, q);
                    const Slot& w = stage[(frag_w_off(kk, lane, wave) + frag_block_off(q)) / 16];
                    if (w.row != kBM + r32 + 32 * q + 128 * (wave >> 1) || w.chunk != chunk)
                        fail("weight fragment reads the wrong row or chunk", lane, kk, q);
                }
    struct Piece { int row = -1, chunk = -1, half = -1; };
    for (int wave = 0; wave < kWaves; ++wave) {
        std::vector<Piece> epi(kEpiWaveB / 8);
        for (int lane = 0; lane < 64; ++lane)
            for (int k = 0; k < 8; ++k) {
                const long long b = (long long)epi_w_piece(epi_w_off(wave, lane), k) - wave * kEpiWaveB;
                in_range("staging write inside the wave's region", b, 8, kEpiWaveB);
                Piece& pc = epi[b / 8];
                if (pc.row >= 0) fail("staging slot written twice", b, lane, k);
                pc = {lane & 31, k, lane >> 5};
            }
        for (int lane = 0; lane < 64; ++lane)
            for (int s4 = 0; s4 < 4; ++s4) {
                const long long b = (long long)epi_r_off(wave, lane) + s4 * 8 * kEpiRowB - wave * kEpiWaveB;
                in_range("staging read inside the wave's region", b, 16, kEpiWaveB);
                Piece lo = epi[b / 8], hi = epi[b / 8 + 1];
#ifndef PLANT_NO_UNSWAP  // a planted mistake: the read-back halves left as stored
                if (epi_r_swapped(s4)) std::swap(lo, hi);
#endif
                const int R = lane / 8 + 8 * s4, c = lane & 7;
                if (lo.row != R || hi.row != R || lo.chunk != c || hi.chunk != c || lo.half != 0 || hi.half != 1)
                    fail("staging read-back holds the wrong row, chunk or half", lane, s4, wave);
                for (int gr = 0; gr < 8; ++gr) {
                    const long long o = bf16_store_off(gr, s4, (int)ncol) + epi_gl_off(lane, (int)ncol);
                    const long long want = ((32LL * (gr >> 1) + R) * ncol + 64 * (gr & 1) + 8 * c) * 2;
                    if (o != want) fail("bf16 store of a read-back goes to the wrong row or channels", lane, s4, gr);
                }
            }
    }
}

void replay(const Launch& L) {
    const bool bf16_out = L.epi == "bf16";
    const bool add = L.epi == "f32add";
    const int out_elem = bf16_out ? 2 : 4;
    const int kStores = bf16_out ? kStoresBf16 : kStoresF32;
    const long long A_bytes = L.M * L.K * L.elem;
    const long long Bt_bytes = L.bt_elems * L.elem;
    const long long plane_bytes = L.M * L.ncol * out_elem;
    const long long row_bytes = L.K * L.elem;
    const int nN = (int)(L.N / kBN);
    const int nk = (int)(L.K / (kSlabB / L.elem));
    const int ntiles = (int)(L.M / kBM) * nN;
    if (L.M % kBM || L.N % kBN || L.ncol % kBN || nk % 4 || L.rows_per_batch % kBM || L.N > L.ncol * L.nplanes)
        fail("shape outside the MFMA kernel's domain", L.M, L.N, L.K);
    check_layouts(row_bytes, L.ncol);
    const int grid = grid_size(ntiles, (int)L.n_cu);
    std::vector<int> visits(ntiles, 0);
    const int y_store = kStores + 2 * kDmaPerSlab <= 63 ? kStores + 2 * kDmaPerSlab : 0;

    for (int block = 0; block < grid; ++block) {
        const Sched sc = schedule(block, grid, ntiles);
        if (sc.tile >= sc.tile_end) continue;
        for (int t = sc.tile; t < sc.tile_end; t += sc.stride) {
            if (t < 0 || t >= ntiles) fail("tile outside the grid of tiles", t, ntiles, block);
            ++visits[t];
        }
        for (int wave = 0; wave < kWaves; ++wave) {
            unsigned vmin = ~0u, vmax = 0;
            for (int lane = 0; lane < 64; ++lane) {
                const unsigned v = dma_lane_off(wave, lane, row_bytes);
                vmin = v < vmin ? v : vmin;
                vmax = v > vmax ? v : vmax;
                in_range("direct-load lane slot in its 1 KiB LDS group", 16 * lane, 16, 1024);
            }
            auto tile_bases = [&](int tile, long long* xb, long long* wb) {
                long long xe, we;
                tile_row_elems(tile, nN, L.K, (int)L.rows_per_batch, L.bt_batch_stride, &xe, &we);
                *xb = xe * L.elem;
                *wb = we * L.elem;
            };
            Wave wv;
            auto issue_slab = [&](int tile, int ks, int st) {
                long long xb, wb;
                tile_bases(tile, &xb, &wb);
                for (int j = 0; j < kDmaPerSlab; ++j) {
                    const long long src = (j < 4 ? xb : wb) + dma_src_off(j, wave, row_bytes, ks);
                    const long long size = j < 4 ? A_bytes : Bt_bytes;
                    in_range(j < 4 ? "direct load from A" : "direct load from Bt", src + vmin, 0, size);
                    in_range(j < 4 ? "direct load from A" : "direct load from Bt", src + vmax, 16, size);
                    in_range("direct load into the LDS ring", (long long)st * kStageB + dma_lds_off(j, wave),
                             1024, (long long)kStages * kStageB);
                    wv.issue({tile, ks});
                }
                wv.stage[st] = {tile, ks};
            };
            // Fragment reads: the same offsets inside whichever stage holds the slab.
            for (int lane = 0; lane < 64; ++lane)
                for (int kk = 0; kk < 2; ++kk)
                    for (int q = 0; q < 4; ++q) {
                        in_range("cell fragment read inside its stage", frag_x_off(kk, lane, wave) + frag_block_off(q), 16, kStageB);
                        in_range("weight fragment read inside its stage", frag_w_off(kk, lane, wave) + frag_block_off(q), 16, kStageB);
                    }
            auto read_slab = [&](int tile, int ks) { wv.read(ks % kStages, {tile, ks}); };
            // Epilogue: per-lane byte offsets from the wave's first output element do not
            // depend on the tile; their range is checked against each tile's base below.
            long long omin = 1LL << 62, omax = -(1LL << 62);
            for (int lane = 0; lane < 64; ++lane) {
                if (bf16_out) {
                    for (int k = 0; k < 8; ++k) {
                        const long long w = epi_w_piece(epi_w_off(wave, lane), k);
                        in_range("epilogue staging write in the wave's region", w - wave * kEpiWaveB, 8, kEpiWaveB);
                    }
                    for (int s4 = 0; s4 < 4; ++s4)
                        in_range("epilogue staging read in the wave's region",
                                 epi_r_off(wave, lane) + s4 * 8 * kEpiRowB - wave * kEpiWaveB, 16, kEpiWaveB);
                    for (int gr = 0; gr < 8; ++gr)
                        for (int s4 = 0; s4 < 4; ++s4) {
                            const long long o = bf16_store_off(gr, s4, (int)L.ncol) + epi_gl_off(lane, (int)L.ncol);
                            omin = o < omin ? o : omin;
                            omax = o > omax ? o : omax;
                        }
                } else {
                    const long long le = f32_lane_elem(lane, (int)L.ncol);
                    for (int j = 0; j < 4; ++j)
                        for (int i = 0; i < 4; ++i)
                            for (int q = 0; q < 4; ++q) {
                                const long long o = (le + f32_store_elem(j, i, q, (int)L.ncol)) * 4;
                                omin = o < omin ? o : omin;
                                omax = o > omax ? o : omax;
                            }
                }
            }

            // Prologue: slabs 0..3 of the first tile, wait for slab 0, read it.
            int tile = sc.tile;
            for (int s = 0; s < 4; ++s) issue_slab(tile, s, s);
            wv.wait(3 * kDmaPerSlab, {tile, 0});
            read_slab(tile, 0);
            bool stores_pending = false;
            while (true) {
                const int next = tile + sc.stride < sc.tile_end ? tile + sc.stride : -1;
                const int y_first = stores_pending ? y_store : 2 * kDmaPerSlab;
                for (int kt = 0; kt < nk; ++kt) {
                    const bool first_group = kt < 4;
                    const int y = (first_group && (kt & 3) < 3) ? y_first : 2 * kDmaPerSlab;
                    const SlabId need = kt + 1 < nk ? SlabId{tile, kt + 1} : SlabId{next >= 0 ? next : tile, 0};
                    wv.wait(y + L.plant, need);
                    const int ks = kt + 4;
                    if (ks < nk) issue_slab(tile, ks, kt % 4);
                    else issue_slab(next >= 0 ? next : tile, ks - nk, kt % 4);
                    if (kt + 1 < nk) read_slab(tile, kt + 1);
                }
                // Epilogue: the tile leaves (and for the adding epilogue its addend is read).
                const int plane = tile_plane(tile, nN, (int)L.ncol);
                if (plane < 0 || plane >= L.nplanes) fail("output plane out of range", plane, tile, L.nplanes);
                const long long wb = wave_out_elem(tile, nN, (int)L.ncol, wave) * out_elem;
                const char* what = bf16_out ? "bf16 store inside its plane"
                                   : add    ? "fp32 store / addend load inside the plane"
                                            : "fp32 store inside its plane";
                in_range(what, wb + omin, 16, plane_bytes);
                in_range(what, wb + omax, 16, plane_bytes);
                for (int i = 0; i < kStores; ++i) wv.issue({-2, -2});
                stores_pending = true;
                if (next < 0) break;
                read_slab(next, 0);
                tile = next;
            }
            wv.drain();  // the kernel's final wait_vm(0)
        }
    }
    for (int t = 0; t < ntiles; ++t)
        if (visits[t] != 1) fail("tile not visited exactly once", t, visits[t], ntiles);
    std::printf("OK grid=%d tiles=%d slabs/tile=%d checks=%lld\n", grid, ntiles, nk, g_checks);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 12 && argc != 13) {
        std::fprintf(stderr, "usage: %s M N K elem rows_per_batch bt_batch_stride bt_elems ncol nplanes n_cu epilogue\n",
                     argv[0]);
        return 2;
    }
    Launch L;
    long long* f[] = {&L.M, &L.N, &L.K, &L.elem, &L.rows_per_batch, &L.bt_batch_stride, &L.bt_elems,
                      &L.ncol, &L.nplanes, &L.n_cu};
    for (int i = 0; i < 10; ++i) *f[i] = std::atoll(argv[1 + i]);
    L.epi = argv[11];
    if (argc == 13) {
        if (std::strcmp(argv[12], "plant-loose-wait") != 0) return 2;
        L.plant = kDmaPerSlab;
    }
    replay(L);
    return 0;
}
