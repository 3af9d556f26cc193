// stencil_sched.hpp — which tiles a workgroup of the bf16 stencil processes.
//
// Workgroup i runs on XCD i % 8 (the dispatcher deals workgroups to the XCDs in
// turn). When the grid and the tile count are multiples of 8, XCD x owns the x-th
// eighth of the tiles ("ticketed" walk): the first `first` tiles of an eighth go one
// to each of the XCD's workgroups, and every later tile is handed out in order by
// the XCD's ticket counter, drawn once per tile by each workgroup. A workgroup whose
// ticket lands past the eighth stops after its current tile and counts itself
// finished on a second counter; the XCD's `first` workgroups are the ones that
// count, and the last of them zeroes both counters for the next launch. Otherwise a
// fixed stride over all tiles.
//
// Plain C++ (no HIP types): the kernel uses these functions, and a host program
// replays the walk in arbitrary orders of the draws (tests/stencil_sched_check.cpp).
#pragma once

#if defined(__HIPCC__)
#define SLIME_SCHED_HD __host__ __device__ __forceinline__
#else
#define SLIME_SCHED_HD inline
#endif

namespace slime {
namespace sched {

struct StencilWalk {
    bool ticketed;
    int xcd, span, first;       // ticketed: XCD, tiles per eighth, fixed tiles per eighth
    int t_cur, t_stride, t_end;  // first tile, fixed stride (0 when ticketed), end of range
};

SLIME_SCHED_HD StencilWalk stencil_walk(int block, int grid, int ntiles) {
    StencilWalk w;
    w.ticketed = (grid & 7) == 0 && (ntiles & 7) == 0;
    w.xcd = block & 7;
    w.span = ntiles >> 3;
    const int nwx = grid >> 3;
    w.first = nwx < w.span ? nwx : w.span;
    if (w.ticketed) {
        w.t_cur = w.xcd * w.span + (block >> 3);
        w.t_stride = 0;
        w.t_end = w.xcd * w.span + w.span;
    } else {
        w.t_cur = block;
        w.t_stride = grid;
        w.t_end = ntiles;
    }
    return w;
}

// A workgroup with t_cur >= t_end has no tile; when ticketed it is not among the
// `first` workgroups that count themselves finished.
SLIME_SCHED_HD bool has_tile(const StencilWalk& w) { return w.t_cur < w.t_end; }

// The fixed-stride successor of tile t, or -1.
SLIME_SCHED_HD int strided_next(const StencilWalk& w, int t) {
    return t + w.t_stride < w.t_end ? t + w.t_stride : -1;
}

// The tile a ticket (the counter's value before the draw) hands out, or -1.
SLIME_SCHED_HD int ticket_tile(const StencilWalk& w, int ticket) {
    return w.first + ticket < w.span ? w.xcd * w.span + w.first + ticket : -1;
}

// The finish count (the counter's value before this workgroup's increment) at which
// this workgroup is the XCD's last and resets the counters.
SLIME_SCHED_HD bool last_finisher(const StencilWalk& w, unsigned finished_before) {
    return finished_before == (unsigned)w.first - 1u;
}

}  // namespace sched
}  // namespace slime
