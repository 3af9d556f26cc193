// Host check of the bf16 stencil's 3x3-kernel operand construction
// (slime_amd/csrc/stencil_band.hpp): for every lane of the Kmat^T operand -- tile cell
// c (0..31), 8-row group grp (0..3), k-step ks (0..1) -- the four dwords built with
// v_perm_b32 from the band table entry of run band_run(c, grp, ks) must equal the
// dense definition Kmat[c][n] = K[3 dy + dx] when n = (c / 8 + dy) * 10 + c % 8 + dx
// (dy, dx < 3), else 0, for halo rows n = 32 ks + 8 grp + e. Test infrastructure: built
// with g++ by tests/test_stencil_band.py; nothing in the library uses it.
//
// Usage: stencil_band_check [plant]   plant = "swap-ab" builds the table with A and B
// exchanged (a planted mistake the check must report).
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../slime_amd/csrc/stencil_band.hpp"

using namespace slime::band;

// v_perm_b32 as the ISA defines it for the selectors used here: byte i of the result
// is byte sel_i of the 64-bit value {s0 (high dword), s1 (low dword)}, or 0 for 0x0C.
static uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    const uint64_t v = (uint64_t)s0 << 32 | s1;
    uint32_t out = 0;
    for (int i = 0; i < 4; ++i) {
        const unsigned s = (sel >> (8 * i)) & 0xff;
        uint32_t b;
        if (s < 8) b = (uint32_t)(v >> (8 * s)) & 0xff;
        else if (s == 0x0C) b = 0;
        else { std::printf("FAIL selector byte %#x outside the forms used\n", s); return 0xdeadbeef; }
        out |= b << (8 * i);
    }
    return out;
}

static uint16_t dense(const uint16_t* k, int c, int n) {
    for (int dy = 0; dy < 3; ++dy)
        for (int dx = 0; dx < 3; ++dx)
            if (n == (c / 8 + dy) * 10 + c % 8 + dx) return k[3 * dy + dx];
    return 0;
}

int main(int argc, char** argv) {
    const bool swap_ab = argc > 1 && std::strcmp(argv[1], "swap-ab") == 0;
    long long checks = 0;
    for (int trial = 0; trial < 4; ++trial) {
        uint16_t k[9];
        uint32_t s = 0x9e3779b9u * (trial + 1);
        for (int i = 0; i < 9; ++i) {
            s = s * 1664525u + 1013904223u;
            k[i] = (uint16_t)((s >> 16) | 1);  // nonzero bf16 bit patterns
        }
        uint32_t table[3][2];
        for (int r = 0; r < 3; ++r) {
            table[r][0] = k[3 * r] | (uint32_t)k[3 * r + 1] << 16;  // A
            table[r][1] = k[3 * r + 2];                             // B
            if (swap_ab) { const uint32_t t = table[r][0]; table[r][0] = table[r][1]; table[r][1] = t; }
        }
        for (int c = 0; c < 32; ++c)
            for (int grp = 0; grp < 4; ++grp)
                for (int ks = 0; ks < 2; ++ks) {
                    const int r = band_run(c, grp, ks);
                    if (r < 0 || r > 2) { std::printf("FAIL run %d out of range\n", r); return 1; }
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t w = perm(table[r][1], table[r][0], band_sel(c, grp, ks, d));
                        for (int h = 0; h < 2; ++h) {
                            const int n = 32 * ks + 8 * grp + 2 * d + h;
                            const uint16_t got = (uint16_t)(w >> (16 * h)), want = dense(k, c, n);
                            ++checks;
                            if (got != want) {
                                std::printf("FAIL cell %d grp %d ks %d halo row %d: %#06x, want %#06x\n", c, grp, ks, n, got, want);
                                return 1;
                            }
                        }
                    }
                }
    }
    // Every weight of every cell reaches some lane (the 9 taps lie in rows 0..63).
    for (int c = 0; c < 32; ++c)
        for (int dy = 0; dy < 3; ++dy)
            for (int dx = 0; dx < 3; ++dx)
                if ((c / 8 + dy) * 10 + c % 8 + dx >= 64) { std::printf("FAIL tap outside the 64 halo rows\n"); return 1; }
    std::printf("OK %lld operand elements\n", checks);
    return 0;
}
