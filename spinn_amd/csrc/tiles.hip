// tiles.hip - output-tile and split-K choice shared by the MFMA GEMM launches.
#include "spinn_hip_internal.h"
#include "streamk.h"
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <mutex>

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

bool tiles_forced() { return g_force_bm != 0 || g_force_split > 1; }

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

int wavek_tile(int M, int N, int K, int reps, WkKind kind) {
    if (g_force_bm) return (g_force_bm == g_force_bn && (g_force_bm == 32 || g_force_bm == 16)) ? g_force_bm : 0;
    const int e = env_wavek();
    if (e >= 0) return e == 1 ? 32 : 0;
    const int cus = device_cu_count();
    const int64_t tiles64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64) * reps;
    // 1x1 convs with K = 64 into one 64-row tile over 1 to 2 tiles per CU: each
    // 64 x 64 tile is four K slices of load, prologue and store, and 16 x 16
    // wave-K tiles stream them instead (64@56x56 at batch 8: 13.7 -> 9.7 us,
    // YOLOv10n's 64@80x80 at batch 4: 13.1 -> 9.1 us); over more tiles (batch 32,
    // 1568) the 64 x 64 tiles keep 16.7 against 28.5 us.
    if (kind == kWkConvPointwise && M <= 64 && K > 48 && K <= 64 && tiles64 < 2 * (int64_t)cus) return 16;
    // and 1x1 convs with K of 96..192 over one to two tiles per CU: 32 x 32 tiles
    // (128 -> 512@28x28 at batch 4: 15.1 -> 13.2 us, YOLOv10n's 128 -> 256@20x20 at
    // batch 16: 15.5 -> 13.3 us; with K = 256 no gain, and below one tile per CU the
    // unsplit 64 x 64 tiles below win)
    if (kind == kWkConvPointwise && K >= 96 && K <= 192 && tiles64 >= cus && tiles64 < 2 * (int64_t)cus) return 32;
    if (tiles64 >= cus) return 0;
    // Measured on MI355X (ResNet-101 and YOLOv10n at batch 1, the Gemm sweep; the
    // batch-1 conv layers with their weights cycled through copies larger than the
    // Infinity Cache, as inside a model).
    // 16 x 16 tiles: 1x1 convs whose 32 x 32 grid covers at most half the CUs with
    // K of 256..1024 (the 1024 -> 256 layers at 14x14: 8.1 -> 5.8 us, split-K's
    // reduction launch gone), and 1x1 convs with K of 64..128 over at most ~1.6
    // 32 x 32 tiles per CU (YOLOv10n 128@20x20: 3.9 -> 2.8 us, 128 -> 512@28x28 of
    // ResNet-101: 5.4 -> 4.6 us; with more tiles, 64 -> 256@56x56, the 64-wide tiles
    // keep 4.7 against 5.8 us). Gathered (3x3) convs with K of 576..1152 over at most
    // ~0.8 16 x 16 tiles per CU: 128@20x20 10.2 -> 6.9 us against split K, 64@20x20
    // 7.9 -> 6.0 us against 32 x 32 tiles; over more tiles (64@40x40, 400) the 32 x 32
    // tiles keep 7.5 against 8.8 us, and a longer gather (256 -> 64@20x20, K = 2304)
    // keeps split K (10.4 against 12.0).
    const int64_t tiles32 = (int64_t)((M + 31) / 32) * ((N + 31) / 32) * reps;
    const int64_t tiles16 = (int64_t)((M + 15) / 16) * ((N + 15) / 16) * reps;
    if (kind == kWkConvPointwise) {
        if (tiles32 <= cus / 2 && K >= 256 && K <= 1024) return 16;
        if (16 * tiles32 <= 25 * (int64_t)cus && K >= 64 && K <= 128) return 16;
        // 32 x 32 tiles for 1x1 convs with K of 577..1152 over at most ~0.43 64 x 64
        // tiles per CU, where the 64 x 64 grid would split K 8 ways (ResNet-101's
        // 1024 -> 256@14x14 at batch 4: 13.3 -> 10.0 us, batch 8: 20.1 -> 15.6 us)
        if (K > 576 && K <= 1152 && 7 * tiles64 <= 3 * (int64_t)cus) return 32;
    }
    if (kind == kWkConvGather && 32 * tiles16 <= 25 * (int64_t)cus && K >= 576 && K <= 1152) return 16;
    // 32 x 32 tiles where 64 x 64 tiles underfill the chip and K is 128..576
    // (one to a few 32-deep chunks per wave); with longer K its one-float-per-lane
    // operand loads cost more than the 64 x 64 tiles' split-K reduction launch,
    // and below 128 it saves nothing. A conv grid of more than half a 64 x 64 tile
    // per CU keeps the 64 x 64 tiles, unsplit (choose_tiles): ResNet-101 at batch 4,
    // 256 -> 1024@14x14 (208 tiles) 10.6 -> 8.4 us, 512 -> 1024@28x28 stride 2
    // 22.0 -> 15.8 us; YOLOv10n at batch 4, 192 -> 128@40x40 9.8 -> 7.0 us.
    if (kind != kWkGemm && 2 * tiles64 > cus) return 0;
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
        ((K >= 512 && 2 * tiles <= cus) || (K >= 1536 && tiles < 2 * cus) || (K >= 256 && 2 * tiles < cus))) {
        // Split K only when each split still runs >= 128 deep: the partial
        // sums cost a write and a read of the output per split. A K of 512
        // or more splits over at most half a tile per CU (a grid of half to
        // one tile per CU runs faster unsplit: ResNet-101's 1024 -> 512@14x14
        // at batch 8, 200 tiles, 27.7 -> 21.9 us with its weights cold, as in
        // a model). A grid of 1-2 tiles per CU splits only a long K (>= 1536: the 3x3 convs of
        // ResNet-101 at batch 32 gain, its 1024-deep 1x1 convs lose); a
        // 256-deep K splits only when the grid covers less than half the
        // CUs (batch-1 1x1 convs). At most 16 splits: measured on the batch-1
        // ResNet-101 convs, 16 beat 8 (the 14x14 3x3 layers then cover all
        // CUs), while 64-deep splits or 8 workgroups per CU were slower; up to
        // 32 where 16 would still leave CUs idle (the 7x7 3x3 layers at batch 1:
        // 8 tiles, K = 4608, 144-deep splits on 256 workgroups).
        int split = (int)std::min<int64_t>((4 * cus + tiles - 1) / tiles, K / 128);
        split = std::max(1, std::min(split, tiles * 16 < cus ? 32 : 16));
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

static int g_force_streamk = -1;
static bool g_force_sys_exchange = false;

void force_streamk(int mode) {
    g_force_streamk = mode < 0 ? -1 : (mode ? 1 : 0);
    g_force_sys_exchange = mode == 2;
}

static int env_streamk() {
    // SPINN_STREAMK=0 never splits the remainder tiles along K, 1 does it for
    // every grid whose tile count is not a multiple of the CU count; unset =
    // per-shape choice.
    static int v = [] {
        const char *e = std::getenv("SPINN_STREAMK");
        if (!e || !*e) return -1;
        return e[0] == '0' ? 0 : 1;
    }();
    return v;
}

bool plan_streamk(int tiles_m, int tiles_n, int S, int tile_elems, SkPlan &p) {
    const int cus = device_cu_count();
    if (cus % kXcds || tiles_m <= 0 || tiles_n <= 0 || S <= 0) return false;
    const int64_t T = (int64_t)tiles_m * tiles_n;
    const int64_t full = T / cus;
    const int R = (int)(T % cus);
    // Fewer tiles than CUs keep split-K or the wave-K kernel: every tile would
    // be cut, and the last part's serial read-back of the others costs more
    // than the reduction launch it saves (measured at batch 1).
    if (R == 0 || full == 0 || T > (int64_t)INT32_MAX / 2) return false;
    const int mode = g_force_streamk >= 0 ? g_force_streamk : env_streamk();
    if (mode == 0 || g_force_split > 1) return false; // a forced K split keeps its grid
    // Whole tiles alone leave full + 1 tiles on the busiest CU against T/C on
    // average: split the remainder when that costs >= 10 % (below that the
    // parts' write-back and read-back cost as much as they save; measured on
    // ResNet-101's batch-32 layers).
    if (mode < 0 && (double)(full + 1) * cus < 1.10 * (double)T) return false;
    const int cx = cus / kXcds;
    const int rx = (R + kXcds - 1) / kXcds;
    p.dp_per_xcd = (int)(full * cx);
    p.R = R;
    p.cnt_bytes = ((size_t)R * 8 + 255) / 256 * 256;
    size_t slots;
    if (full <= 2 && 4 * R > cus) {
        // One extra workgroup per CU (beside at most two whole ones) takes an
        // equal range of the remaining slices; with at least one workgroup per
        // remaining tile of an XCD a range spans at most two tiles.
        p.scheme = kSkSplitWgs;
        p.W = std::max(cx, rx);
        p.p = 0;
        slots = (size_t)kXcds * p.W * 2;
    } else {
        // Parts of >= 4 slices, at most one per CU, done by whole-tile
        // workgroups before their own tile.
        p.scheme = kSkPartsInDp;
        p.W = 0;
        p.p = std::min(std::min(cx / rx, S / 4), kSkMaxParts);
        if (p.p < 2) return false;
        slots = (size_t)kXcds * rx * p.p;
    }
    p.grid = kXcds * p.W + kXcds * p.dp_per_xcd;
    p.ws_bytes = p.cnt_bytes + slots * (size_t)tile_elems * sizeof(float);
    return true;
}

// One workgroup thread records the XCD it runs on (hardware register XCC_ID).
__global__ void xcc_id_kernel(unsigned *out, int n) {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    if (threadIdx.x == 0 && (int)blockIdx.x < n) out[blockIdx.x] = v & 0xFu;
}

namespace {
constexpr int kMaxDevices = 64;
struct XcdState {
    std::once_flag once;
    std::atomic<int> local{0};
};
XcdState g_xcd[kMaxDevices];

// Launch xcc_id_kernel over 4096 workgroups on a private stream and check that
// block id b ran on XCD b % 8. Relaxed capture mode lets the check run even
// while this thread captures a graph on another stream.
int probe_xcd_mapping() {
    constexpr int n = 4096;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return 0;
    int ok = 0;
    unsigned *d = nullptr;
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess &&
        hipMalloc((void **)&d, n * sizeof(unsigned)) == hipSuccess) {
        unsigned h[n];
        hipLaunchKernelGGL(xcc_id_kernel, dim3(n), dim3(64), 0, st, d, n);
        if (hipGetLastError() == hipSuccess &&
            hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, st) == hipSuccess &&
            hipStreamSynchronize(st) == hipSuccess) {
            ok = 1;
            for (int i = 0; i < n && ok; ++i) ok = h[i] == (unsigned)(i % kXcds);
        }
    }
    if (d) (void)hipFree(d);
    if (st) (void)hipStreamDestroy(st);
    (void)hipGetLastError();
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    return ok;
}
} // namespace

void probe_xcd_local(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    XcdState &x = g_xcd[device];
    std::call_once(x.once, [&x]() { x.local.store(probe_xcd_mapping()); });
}

bool xcd_local_parts() {
    if (g_force_sys_exchange) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    return g_xcd[dev].local.load() != 0;
}

namespace {
std::once_flag g_status_once;
unsigned *g_status_host = nullptr; // pinned host word
unsigned *g_status_dev = nullptr;  // its device address
std::atomic<int> g_sk_tries{4};
} // namespace

void init_device_status() {
    std::call_once(g_status_once, []() {
        void *h = nullptr;
        if (hipHostMalloc(&h, sizeof(unsigned), hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        *(volatile unsigned *)h = 0u;
        void *d = nullptr;
        if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
            (void)hipGetLastError();
            d = h;
        }
        g_status_host = (unsigned *)h;
        g_status_dev = (unsigned *)d;
    });
}

unsigned *device_status_word() { return g_status_dev; }

int take_device_status() {
    if (!g_status_host) return 0;
    volatile unsigned *w = g_status_host;
    const unsigned v = *w;
    if (v) *w = 0u;
    return (int)v;
}

void force_streamk_tries(int tries) { g_sk_tries.store(tries < 0 ? 4 : tries); }
int streamk_tries() { return g_sk_tries.load(); }

uint64_t streamk_epoch() {
    // 48-bit launch tags, never 0; the start varies between processes.
    static std::atomic<uint64_t> next{(uint64_t)std::chrono::steady_clock::now().time_since_epoch().count() * 2654435761u};
    uint64_t e = next.fetch_add(1) & ((1ull << 48) - 1);
    return e ? e : 1;
}

} // namespace spinn
