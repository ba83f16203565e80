// Tile schedule shared by the persistent GEMM kernels (host + device, so the
// host-side schedule check in tests/sched_check.hip exercises this exact code).
#pragma once

#include <stdint.h>

#include "lsmx_common.h"

namespace lsmx {

LSMX_HD int imin(int a, int b) { return a < b ? a : b; }
LSMX_HD int imax(int a, int b) { return a > b ? a : b; }

// Map a linear tile id to a (tile_m, tile_n) pair.  Consecutive workgroup ids
// are dispatched round-robin over the 8 XCDs; the remap hands each XCD a run
// of consecutive logical tiles, and groups of `group_m` tile rows keep the A
// and B panels those tiles share resident in that XCD's L2.  Ids outside
// [0, tiles) are clamped to that range, so every result indexes a real tile.
LSMX_HD void tile_coords(int pid, int tiles_m, int tiles_n, int group_m, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    pid = imax(0, imin(pid, total - 1));
    if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
    const int per_group = group_m * tiles_n;
    const int group = pid / per_group;
    const int first_m = group * group_m;
    const int gsz = imin(tiles_m - first_m, group_m);
    const int in_group = pid - group * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

// Unsigned division by a divisor fixed for the whole kernel, with no divide
// instruction: m = floor((2^32 - 1) / d) makes mul_hi(n, m) equal n / d or
// n / d - 1 (m*d <= 2^32 - 1 and m*d > 2^32 - 1 - d), so one compare fixes it.
// Exact for every 32-bit n and d >= 1; on the GPU it is scalar code when n
// and d are wave-uniform.
struct DivU32 {
    uint32_t d, m;
};
LSMX_HD DivU32 make_div(uint32_t d) { return DivU32{d, 0xFFFFFFFFu / d}; }
LSMX_HD uint32_t udiv(uint32_t n, DivU32 v) {
    uint32_t q = (uint32_t)(((uint64_t)n * v.m) >> 32);
    if (n - q * v.d >= v.d) ++q;
    return q;
}

// tile_coords with the divisions by the group stride and the group height
// replaced by udiv: what the persistent kernels evaluate in their main loop.
struct TileMap {
    int tiles_m, tiles_n, total, group_m;
    DivU32 per_group;
};
LSMX_HD TileMap make_tile_map(int tiles_m, int tiles_n, int group_m) {
    return TileMap{tiles_m, tiles_n, tiles_m * tiles_n, group_m, make_div((uint32_t)(group_m * tiles_n))};
}
// The group-of-rows part of tile_coords alone, for an id already remapped
// per XCD (or deliberately not remapped); id in [0, total).
LSMX_HD void group_coords(int pid, const TileMap &t, int &tm, int &tn) {
    const int group = (int)udiv((uint32_t)pid, t.per_group);
    const int first_m = group * t.group_m;
    const int gsz = imin(t.tiles_m - first_m, t.group_m);
    const int in_group = pid - group * (int)t.per_group.d;
    // gsz is 1..group_m (at most 4 here): m = floor((2^32 - 1) / gsz)
    const uint32_t gm = (gsz == 3 ? 0x55555555u : 0u) | (gsz != 3 ? 0xFFFFFFFFu >> (gsz >> 1) : 0u);
    const int q = (int)udiv((uint32_t)in_group, DivU32{(uint32_t)gsz, gm});
    tm = first_m + (in_group - q * gsz);
    tn = q;
}
LSMX_HD void tile_coords(int pid, const TileMap &t, int &tm, int &tn) {
    // written without branches so that it stays inside one basic block of a
    // kernel's main loop (the scheduling fences there only act within one)
    pid = imax(0, imin(pid, t.total - 1));
    const int xcd = (pid & 7) * (t.total >> 3) + (pid >> 3);
    pid = (t.total & 7) == 0 ? xcd : pid;
    group_coords(pid, t, tm, tn);
}

// Number of tiles a persistent workgroup `wg` of `grid` processes.
LSMX_HD int tiles_of_workgroup(int tiles, int wg, int grid) { return (tiles - wg + grid - 1) / grid; }

// The tile (as an iteration index of workgroup `wg`, clamped to its last real
// tile) that holds pipeline stage u when each tile has nk stages.  Stages
// beyond the workgroup's work are prefetch refills whose data is never read;
// clamping keeps their addresses inside the operands.
LSMX_HD int stage_tile_iter(int u, int nk, int my_tiles) { return imin(u / nk, my_tiles - 1); }

}  // namespace lsmx
