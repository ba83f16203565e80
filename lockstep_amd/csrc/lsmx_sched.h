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

// Number of tiles a persistent workgroup `wg` of `grid` processes.
LSMX_HD int tiles_of_workgroup(int tiles, int wg, int grid) { return (tiles - wg + grid - 1) / grid; }

// The tile (as an iteration index of workgroup `wg`, clamped to its last real
// tile) that holds pipeline stage u when each tile has nk stages.  Stages
// beyond the workgroup's work are prefetch refills whose data is never read;
// clamping keeps their addresses inside the operands.
LSMX_HD int stage_tile_iter(int u, int nk, int my_tiles) { return imin(u / nk, my_tiles - 1); }

}  // namespace lsmx
