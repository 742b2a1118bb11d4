// tiles.hip - output-tile and split-K choice shared by the MFMA GEMM launches.
#include "spinn_hip_internal.h"

namespace spinn {

// Pick the output tile and K split for an (M x N) problem repeated `reps`
// times (groups or batch). Larger tiles do more MFMA work per byte staged,
// but a launch needs enough workgroups to occupy every CU (2 resident per CU).
TileChoice choose_tiles(int M, int N, int K, int reps, bool allow_split) {
    static const int cand[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
    const int cus = device_cu_count();
    double best = 1e300;
    TileChoice tc{64, 64, 1, K};
    for (auto &c : cand) {
        const int bm = c[0], bn = c[1];
        const int64_t tiles = (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * reps;
        // Each CU works through ceil(tiles / CUs) tiles; a tile costs bm*bn*K
        // MFMA work at an efficiency that drops for smaller tiles (more bytes
        // staged per flop, fewer MFMAs per barrier).
        const double tile_eff = (bm == 128 && bn == 128) ? 1.0 : (bm * bn == 128 * 64 ? 0.92 : 0.80);
        const double rounds = (double)((tiles + cus - 1) / cus);
        const double est = rounds * bm * bn / tile_eff;
        if (est < best - 1e-9) {
            best = est;
            tc = TileChoice{bm, bn, 1, K};
        }
    }
    if (allow_split) {
        const int64_t tiles = (int64_t)((M + tc.bm - 1) / tc.bm) * ((N + tc.bn - 1) / tc.bn) * reps;
        if (tiles < cus && K >= 4 * kBK * 2) {
            int split = (int)std::min<int64_t>((cus + tiles - 1) / tiles, K / (4 * kBK));
            split = std::max(1, std::min(split, 32));
            if (split > 1) {
                int chunk = (K + split - 1) / split;
                chunk = (chunk + kBK - 1) / kBK * kBK;
                split = (K + chunk - 1) / chunk;
                tc.split = split;
                tc.k_chunk = chunk;
            }
        }
    }
    return tc;
}

} // namespace spinn
