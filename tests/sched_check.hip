// Host-only check of the persistent GEMM tile schedule (lockstep_amd/csrc/lsmx_sched.h).
//
// Replays, for many shapes and grid sizes, the stage sequence the f4 x f4 GEMM
// kernel walks (stages of 64 or 128 bytes per row, rings of 2-4 slots) --
// prologue refills of stages 0..S-1, then per stage the refill of stage
// u + S in the two-phase form the kernels use -- and checks that
//   * every tile is computed by exactly one (workgroup, iteration) pair,
//   * every stage's tile iteration clamps into [0, my_tiles), its tile origin
//     lies inside the operands, and its K offset stays inside a row,
// so no direct-to-LDS load can address memory outside A, B or their scales.
// Built and run on the CPU by tests/test_sched.py; exits non-zero on failure.
#include <cstdio>
#include <vector>

#include "../lockstep_amd/csrc/lsmx_sched.h"

static int failures = 0;
#define CHECK(c, ...)                                    \
    do {                                                 \
        if (!(c)) {                                      \
            if (failures < 10) fprintf(stderr, __VA_ARGS__); \
            ++failures;                                  \
        }                                                \
    } while (0)

static void check_shape(long M, long N, long K, int grid_cap, int S, int group_m, int BM, int BN, int bkb) {
    const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int grid = tiles < grid_cap ? tiles : grid_cap;
    const int nk = (int)(K / (2 * bkb));  // stages per tile: bkb bytes of each row per stage
    std::vector<int> seen(tiles, 0);
    for (int wg = 0; wg < grid; ++wg) {
        const int my_tiles = lsmx::tiles_of_workgroup(tiles, wg, grid);
        auto origin = [&](int ti, long &m0, long &n0) {  // mirrors the kernel's tile_of
            ti = lsmx::imax(0, lsmx::imin(ti, my_tiles - 1));
            int tm, tn;
            lsmx::tile_coords(wg + ti * grid, tiles_m, tiles_n, group_m, tm, tn);
            CHECK(tm >= 0 && tm < tiles_m && tn >= 0 && tn < tiles_n,
                  "bad tile (%d,%d) M=%ld N=%ld wg=%d ti=%d\n", tm, tn, M, N, wg, ti);
            m0 = (long)tm * BM;
            n0 = (long)tn * BN;
        };
        auto check_stage = [&](int ti, int kt) {
            long m0, n0;
            origin(ti, m0, n0);
            CHECK(m0 >= 0 && m0 < M && n0 >= 0 && n0 < N, "origin out of range M=%ld N=%ld\n", M, N);
            CHECK(kt >= 0 && kt < nk, "k-step %d out of range (nk=%d)\n", kt, nk);
            const long last_row_a = lsmx::imin((int)(m0 + BM - 1), (int)(M - 1));
            const long last_row_b = lsmx::imin((int)(n0 + BN - 1), (int)(N - 1));
            CHECK(last_row_a < M && last_row_b < N, "row overflow\n");
            CHECK((long)kt * bkb + bkb <= K / 2, "K offset past the row\n");
        };
        // the kernels' division-free mapping agrees with the reference one
        const lsmx::TileMap tmap = lsmx::make_tile_map(tiles_m, tiles_n, group_m);
        for (int ti = 0; ti < my_tiles + 2; ++ti) {
            int tm0, tn0, tm1, tn1;
            lsmx::tile_coords(wg + ti * grid, tiles_m, tiles_n, group_m, tm0, tn0);
            lsmx::tile_coords(wg + ti * grid, tmap, tm1, tn1);
            CHECK(tm0 == tm1 && tn0 == tn1, "TileMap disagrees at pid %d (M=%ld N=%ld)\n", wg + ti * grid, M, N);
        }
        // computed tiles
        for (int ti = 0; ti < my_tiles; ++ti) {
            long m0, n0;
            origin(ti, m0, n0);
            ++seen[(m0 / BM) * tiles_n + n0 / BN];
        }
        // prologue refills
        for (int p = 0; p < S; ++p) check_stage(lsmx::stage_tile_iter(p, nk, my_tiles), p % nk);
        // steady-state refills, as the kernels walk them: stage kt of tile
        // iteration ti refills k-step kt + ra of tile ti + qa (phase A,
        // kt < nk - ra) or k-step kt + ra - nk of tile ti + qa + 1 (phase B),
        // qa = S / nk, ra = S % nk -- which must be stage u + S, u = ti*nk + kt
        const int qa = S / nk, ra = S % nk;
        for (int ti = 0; ti < my_tiles; ++ti)
            for (int kt = 0; kt < nk; ++kt) {
                const bool pb = kt >= nk - ra;
                const int rt = ti + qa + (pb ? 1 : 0), rk = pb ? kt + ra - nk : kt + ra;
                const int u = ti * nk + kt;
                CHECK(rt == (u + S) / nk && rk == (u + S) % nk, "phase refill (%d,%d) is not stage u+S\n", rt, rk);
                check_stage(rt, rk);
            }
    }
    for (int t = 0; t < tiles; ++t) CHECK(seen[t] == 1, "tile %d computed %d times (M=%ld N=%ld grid=%d)\n", t, seen[t], M, N, grid);
}

// udiv against the divide instruction on edge values and a sweep
static void check_udiv() {
    const uint32_t ds[] = {1, 2, 3, 4, 5, 7, 12, 31, 32, 96, 128, 1000, 4096, 65535, 65536, 123457, 1u << 20,
                           (1u << 31) - 1, 1u << 31, 0xFFFFFFFEu, 0xFFFFFFFFu};
    const uint32_t ns[] = {0, 1, 2, 3, 63, 64, 65, 1000, 65535, 65536, 1u << 20, (1u << 31) - 1, 1u << 31,
                           0xFFFFFFFEu, 0xFFFFFFFFu};
    for (uint32_t d : ds) {
        const lsmx::DivU32 v = lsmx::make_div(d);
        for (uint32_t n : ns) {
            for (uint32_t dn : {0u, 1u, d - 1, d, d + 1}) {
                const uint32_t x = n + dn;
                CHECK(lsmx::udiv(x, v) == x / d, "udiv(%u, %u) = %u, want %u\n", x, d, lsmx::udiv(x, v), x / d);
            }
        }
        for (uint32_t x = 0; x < 200000; x += 7) CHECK(lsmx::udiv(x, v) == x / d, "udiv(%u, %u)\n", x, d);
    }
}

int main() {
    check_udiv();
    const long sizes[] = {1, 2, 31, 37, 128, 255, 256, 257, 300, 513, 1000, 1024, 2048, 4096, 8192, 14336, 16384};
    const long ks[] = {128, 256, 384, 512, 4096};
    const int caps[] = {1, 3, 8, 80, 256, 304};
    int shapes = 0;
    for (long M : sizes)
        for (long N : sizes)
            for (long K : ks)
                for (int cap : caps)
                    for (int S : {2, 3, 4})
                        for (int bkb : {64, 128}) {
                            if (K % (2 * bkb)) continue;  // the kernel takes 128-byte stages only when K % 256 == 0
                            check_shape(M, N, K, cap, S, 4, 256, 256, bkb);
                            ++shapes;
                        }
    printf("schedule check: %d configurations, %d failures\n", shapes, failures);
    return failures ? 1 : 0;
}
