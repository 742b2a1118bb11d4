// tiles.hip - output-tile and split-K choice shared by the MFMA GEMM launches.
#include "spinn_hip_internal.h"
#include <cstdlib>

namespace spinn {

// Pick the output tile and K split for an (M x N) problem repeated `reps`
// times (groups or batch). Larger tiles do more MFMA work per byte staged,
// but a launch needs enough workgroups to occupy every CU (2 resident per CU).
static int g_force_bm = 0, g_force_bn = 0, g_force_split = 0;

void force_tiles(int bm, int bn, int split) {
    g_force_bm = bm;
    g_force_bn = bn;
    g_force_split = split;
}

static int env_wavek() {
    // SPINN_WAVEK=0 never runs the wave-K kernel, 1 runs it for every shape;
    // unset = per-shape choice.
    static int v = [] {
        const char *e = std::getenv("SPINN_WAVEK");
        if (!e || !*e) return -1;
        return e[0] == '0' ? 0 : 1;
    }();
    return v;
}

int wavek_tile(int M, int N, int K, int reps, bool pointwise) {
    if (g_force_bm) return (g_force_bm == g_force_bn && (g_force_bm == 32 || g_force_bm == 16)) ? g_force_bm : 0;
    const int e = env_wavek();
    if (e >= 0) return e == 1 ? 32 : 0;
    const int cus = device_cu_count();
    const int64_t tiles64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64) * reps;
    if (tiles64 >= cus) return 0;
    // Measured on MI355X (ResNet-101 and YOLOv10n at batch 1, the Gemm sweep).
    // 16 x 16 tiles: 1x1 convs whose 32 x 32 grid covers at most half the CUs with
    // K of 256..1024 (the 1024 -> 256 layers at 14x14: 8.1 -> 5.8 us, split-K's
    // reduction launch gone). Their B loads are one float per k and lane, so a
    // 3x3 gather or a longer K stays on 32-wide or split-K tiles.
    const int64_t tiles32 = (int64_t)((M + 31) / 32) * ((N + 31) / 32) * reps;
    if (pointwise && tiles32 <= cus / 2 && K >= 256 && K <= 1024) return 16;
    // 32 x 32 tiles where 64 x 64 tiles underfill the chip and K is 128..576
    // (one to a few 32-deep chunks per wave); with longer K its one-float-per-lane
    // operand loads cost more than the 64 x 64 tiles' split-K reduction launch,
    // and below 128 it saves nothing.
    return (K >= 128 && K <= 576) ? 32 : 0;
}

static bool valid_tile(int bm, int bn) {
    return ((bm == 64 || bm == 128) && (bn == 64 || bn == 128)) || (bm == 32 && bn == 128);
}

TileChoice choose_tiles(int M, int N, int K, int reps, bool allow_split) {
    if (g_force_bm && valid_tile(g_force_bm, g_force_bn)) {
        TileChoice tc{g_force_bm, g_force_bn, 1, K};
        if (allow_split && g_force_split > 1) {
            int chunk = (K + g_force_split - 1) / g_force_split;
            chunk = (chunk + kBK - 1) / kBK * kBK;
            tc.split = (K + chunk - 1) / chunk;
            tc.k_chunk = chunk;
            if (tc.split <= 1) tc.k_chunk = K;
        }
        return tc;
    }
    const int cus = device_cu_count();
    const int64_t work = (int64_t)M * N * reps;
    TileChoice tc{64, 64, 1, K};
    if (work >= (int64_t)64 * cus * 128 * 128) {
        // Large problems (>= 64 full 128x128 tiles per CU): the bigger tile
        // stages half the bytes per flop and still fills the machine.
        tc.bm = tc.bn = 128;
        return tc;
    }
    // At most 32 rows (output channels): a 32 x 128 tile, waves side by side,
    // instead of a 64-row tile that would compute on zero-padded rows.
    // Otherwise 64x64 tiles run up to six blocks per CU, which is what hides
    // the load latency of a short K loop (measured faster than 128-wide tiles
    // on every ResNet-101 layer shape at batch 32).
    if (M <= 32) {
        tc.bm = 32;
        tc.bn = 128;
    }
    const int64_t tiles = (int64_t)((M + tc.bm - 1) / tc.bm) * ((N + tc.bn - 1) / tc.bn) * reps;
    if (allow_split &&
        ((K >= 512 && tiles < cus) || (K >= 1536 && tiles < 2 * cus) || (K >= 256 && 2 * tiles < cus))) {
        // Split K only when each split still runs >= 128 deep: the partial
        // sums cost a write and a read of the output per split. A grid of
        // 1-2 tiles per CU splits only a long K (>= 1536: the 3x3 convs of
        // ResNet-101 at batch 32 gain, its 1024-deep 1x1 convs lose); a
        // 256-deep K splits only when the grid covers less than half the
        // CUs (batch-1 1x1 convs). At most 16 splits: measured on the batch-1
        // ResNet-101 convs, 16 beat 8 (the 14x14 3x3 layers then cover all
        // CUs), while 64-deep splits or 8 workgroups per CU were slower.
        int split = (int)std::min<int64_t>((4 * cus + tiles - 1) / tiles, K / 128);
        split = std::max(1, std::min(split, 16));
        if (split > 1) {
            int chunk = (K + split - 1) / split;
            chunk = (chunk + kBK - 1) / kBK * kBK;
            tc.split = (K + chunk - 1) / chunk;
            tc.k_chunk = chunk;
            if (tc.split <= 1) {
                tc.split = 1;
                tc.k_chunk = K;
            }
        }
    }
    return tc;
}

} // namespace spinn
