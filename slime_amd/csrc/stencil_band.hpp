// stencil_band.hpp — the 3x3 kernel operand of the bf16 stencil's potential sum
// U^T = X_halo^T . Kmat^T, built in registers from a 12-dword table per (pod, head)
// instead of loaded from a dense [32 cells][64 halo rows] matrix.
//
// Kmat[c][n] = K[3 dy + dx] when halo row n = base(c) + 10 dy + dx (dy, dx < 3;
// base(c) = 10 (c / 8) + c % 8 on the 6x10 halo of a 4x8 tile), else 0. Along n a
// cell's row is therefore the 23-element pattern  K0 K1 K2 0*7 K3 K4 K5 0*7 K6 K7 K8
// shifted by base(c). A lane of the MFMA's B operand holds 8 consecutive halo rows
// (32 ks + 8 grp .. +7) of one cell, and since the runs of three are 10 apart, those
// 8 rows meet at most one run r. The lane takes the run's three weights from the
// table entry {A_r, B_r} = {K[3r] | K[3r+1] << 16, K[3r+2]} (bf16 bits) with one
// v_perm_b32 per dword, the byte selectors depending only on the lane (band_sel).
// The weights enter as bf16 hi + lo pairs, so the table holds {A_hi, B_hi, A_lo, B_lo}
// per run: 12 dwords per (pod, head).
//
// Plain C++ (no HIP types) so that a host test checks the selectors against the
// dense definition.
#pragma once

#if defined(__HIPCC__)
#define SLIME_BAND_HD __host__ __device__ __forceinline__
#else
#define SLIME_BAND_HD inline
#endif

namespace slime {
namespace band {

constexpr int kTileX = 8, kHaloX = 10;
constexpr int kZeroSel = 0x0C;  // v_perm_b32 byte selector of a zero byte

// Position of halo row n in cell c's 23-element pattern (negative or >= 23: outside).
SLIME_BAND_HD int pattern_pos(int cell, int n) { return n - ((cell / kTileX) * kHaloX + cell % kTileX); }

// The run (kernel row 0..2) that the 8 rows 32 ks + 8 grp .. +7 of cell c meet, or 0
// when they meet none (the selectors are then all zero).
SLIME_BAND_HD int band_run(int cell, int grp, int ks) {
    for (int e = 0; e < 8; ++e) {
        const int p = pattern_pos(cell, 32 * ks + 8 * grp + e);
        if (p >= 0 && p < 23 && p % 10 < 3) return p / 10;
    }
    return 0;
}

// v_perm_b32 selector of dword d (elements 2d, 2d+1) of that lane's operand, over the
// 8 bytes {B_r (bytes 4..7), A_r (bytes 0..3)}: weight q of the run sits in bytes 2q, 2q+1.
SLIME_BAND_HD unsigned band_sel(int cell, int grp, int ks, int d) {
    unsigned sel = 0;
    for (int half = 0; half < 2; ++half) {
        const int p = pattern_pos(cell, 32 * ks + 8 * grp + 2 * d + half);
        const bool on = p >= 0 && p < 23 && p % 10 < 3;
        const unsigned lo = on ? (unsigned)(2 * (p % 10)) : (unsigned)kZeroSel;
        const unsigned hi = on ? (unsigned)(2 * (p % 10) + 1) : (unsigned)kZeroSel;
        sel |= (lo | (hi << 8)) << (16 * half);
    }
    return sel;
}

}  // namespace band
}  // namespace slime
