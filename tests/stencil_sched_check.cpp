// Host replay of the bf16 stencil's tile walk (slime_amd/csrc/stencil_sched.hpp).
//
// Every workgroup of a launch is simulated: a ticketed workgroup draws a ticket
// from its XCD's counter at the start of each tile and takes the tile the ticket
// hands out after it; when that is none it counts itself finished, and the XCD's
// last finisher zeroes both counters. The draws and finishes of all workgroups are
// interleaved in a seeded random order (any order the device could produce). Two
// launches run back to back on the same counters. Checks: every tile is processed
// exactly once per launch, inside [0, ntiles) and, when ticketed, inside the
// workgroup's own XCD eighth; every counter is zero after each launch.
//
// -DPLANT_FIRST: the tickets start one tile late (a tile is skipped), which the
// check must report.
#include "../slime_amd/csrc/stencil_sched.hpp"

#include <cstdio>
#include <random>
#include <vector>

using namespace slime::sched;

namespace {

struct Wg {
    StencilWalk w;
    int cur;   // tile in progress, -1 when done
    bool counted;
};

int ticket_tile_checked(const StencilWalk& w, int ticket) {
#ifdef PLANT_FIRST
    StencilWalk p = w;
    p.first += 1;
    return ticket_tile(p, ticket);
#else
    return ticket_tile(w, ticket);
#endif
}

// One launch; returns the number of errors.
int launch(int grid, int ntiles, unsigned (&ctr)[16], std::mt19937& rng, const char* name) {
    int errors = 0;
    std::vector<int> seen(ntiles, 0);
    std::vector<Wg> wgs(grid);
    std::vector<int> active;
    for (int b = 0; b < grid; ++b) {
        wgs[b].w = stencil_walk(b, grid, ntiles);
        wgs[b].counted = wgs[b].w.ticketed && has_tile(wgs[b].w);
        wgs[b].cur = has_tile(wgs[b].w) ? wgs[b].w.t_cur : -1;
        if (wgs[b].cur >= 0) active.push_back(b);
    }
    while (!active.empty()) {
        const size_t pick = rng() % active.size();
        Wg& g = wgs[active[pick]];
        const StencilWalk& w = g.w;
        const int t = g.cur;
        if (t < 0 || t >= ntiles) {
            if (errors++ < 5) std::printf("%s: tile %d out of range\n", name, t);
        } else {
            seen[t] += 1;
            if (w.ticketed && (t < w.xcd * w.span || t >= w.xcd * w.span + w.span))
                if (errors++ < 5) std::printf("%s: tile %d outside XCD %d's eighth\n", name, t, w.xcd);
        }
        int next;
        if (w.ticketed) {
            const int ticket = (int)ctr[w.xcd]++;
            next = ticket_tile_checked(w, ticket);
        } else {
            next = strided_next(w, t);
        }
        g.cur = next;
        if (next < 0) {
            if (g.counted) {
                const unsigned before = ctr[8 + w.xcd]++;
                if (last_finisher(w, before)) ctr[w.xcd] = ctr[8 + w.xcd] = 0u;
            }
            active[pick] = active.back();
            active.pop_back();
        }
    }
    for (int t = 0; t < ntiles; ++t)
        if (seen[t] != 1 && errors++ < 5) std::printf("%s: tile %d processed %d times\n", name, t, seen[t]);
    for (int i = 0; i < 16; ++i)
        if (ctr[i] != 0u && errors++ < 5) std::printf("%s: counter %d left at %u\n", name, i, ctr[i]);
    return errors;
}

}  // namespace

int main() {
    // (grid, ntiles): the c3 launch on 256 CUs, the test shapes, grids as large as the
    // tile count, grids that are not multiples of 8 and tile counts that are not.
    const int cases[][2] = {{512, 32768}, {512, 768}, {512, 512}, {160, 768}, {512, 1000},
                            {8, 8},       {16, 24},   {504, 2016}, {510, 4096}, {512, 4100},
                            {80, 80},     {64, 4096}, {7, 100},    {1, 3}};
    int errors = 0;
    std::mt19937 rng(12345);
    for (const auto& c : cases) {
        char name[64];
        std::snprintf(name, sizeof name, "grid %d, %d tiles", c[0], c[1]);
        unsigned ctr[16] = {};
        for (int rep = 0; rep < 2; ++rep)  // two launches on the same counters
            for (int order = 0; order < 3; ++order) errors += launch(c[0], c[1], ctr, rng, name);
    }
    std::printf("%s: %d errors\n", errors ? "FAIL" : "OK", errors);
    return errors ? 1 : 0;
}
