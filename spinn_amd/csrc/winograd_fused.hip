// winograd_fused.hip - F(4x4,3x3) Winograd convolution in one launch, for layers whose
// transform-domain tensors would dwarf the work: few channels over many tiles.
//
// The three-launch form (winograd.hip) writes V = B^T d B for every (channel, tile)
// and M = U V for every (output channel, tile) to memory, 2.25x the input and 2.25x
// the output each, and reads both back; for 64 channels at 56x56 and batch 32 that
// is 230 MB around 1.85 GFLOP of MFMA work. Here one workgroup owns 32 output
// channels x 32 tiles and keeps all 36 transform positions of that block on chip:
//   - input transform: per slice of 4 channels, two threads per (channel, tile)
//     each gather three columns of the 6x6 patch (zero outside the image) and
//     transform them (B^T d), exchange through LDS, and transform three rows each
//     ((B^T d) B: the same values as the three-launch path) into an LDS slice
//     V[36][4][32]; the next slice's patches are loaded while the current slice's
//     MFMAs run (two V slices);
//   - the 36 GEMMs: each wave owns 9 positions and keeps their 32x32 accumulators in
//     registers; A = a U slice [36][4][32] staged in LDS beside the V slice (loaded
//     one K slice ahead, like the patches), B = the V slice; v_mfma_f32_32x32x2f32;
//   - output transform: the accumulators go through LDS in four rounds of 8 output
//     channels (all 36 positions each), and one thread per (output channel, tile)
//     applies Y = A^T M A, then bias, residual and the activation
//     (SPINN/run_time/ops/mm/gemm_kernel.c:316-338), and stores the 4x4 tile.
// No workspace; U is the three-launch path's packing [36][C][OC].
//
// v_mfma_f32_32x32x2f32 register layout: A lane l = A[l%32][k = l/32], B lane l =
// B[k = l/32][l%32], accumulator element r of lane l = D[8*(r/4) + 4*(l/32) + r%4][l%32];
// here M = output channels, N = tiles, K = input channels.
#include "mfma_core.h"
#include "spinn_hip_internal.h"
#include "winograd_tf.h"
#include <cstdlib>

namespace spinn {

namespace {

constexpr int kWfT = 32;                  // tiles per workgroup (MFMA N)
constexpr int kWfCs = 4;                  // channels per K slice (2 MFMA steps)
constexpr int kWfP = 36;                  // transform positions
constexpr int kWfUnits = 9;               // positions per wave (9 * 4 waves = 36)
constexpr int kWfSlice = kWfP * kWfCs * kWfT; // floats of one LDS slice of V (or of the exchange area)

struct WfGeom {
    int C, H, W, OC, OH, OW, PH, PW, TH, TW;
    int T;            // tiles: N * TH * TW
    uint32_t x_bytes; // extent of x
    uint32_t u_bytes; // extent of U (36 * C * OC floats)
};

// One workgroup: 32 output channels x 32 tiles, all 36 positions; 4 waves, wave w owns
// positions 9w .. 9w + 8. LDS: two V slices [36][4][32], an exchange area and a U
// slice of the same size (74 KB: two workgroups per CU).
template <int AC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void wino4_fused_kernel(
    const float *__restrict__ x, const float *__restrict__ U, const float *__restrict__ bias,
    const float *__restrict__ res, float *__restrict__ y, WfGeom g, int vec_out) {
    __shared__ __attribute__((aligned(16))) float lds[4 * kWfSlice];
    float *const vs0 = lds;                 // V slice, even K slices
    float *const vs1 = lds + kWfSlice;      // V slice, odd K slices
    float *const xch = lds + 2 * kWfSlice;  // column-transformed half patches
    float *const us = lds + 3 * kWfSlice;   // U slice [36][4][32] of the current K slice
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int t0 = blockIdx.x * kWfT;
    const int oc0 = blockIdx.y * 32;
    const int S = (g.C + kWfCs - 1) / kWfCs;

    // This thread's tile (the transform and output phases both index tiles by tid % 32).
    const int tl = tid & (kWfT - 1);
    const int t = t0 + tl;
    const bool tv = t < g.T;
    int n = 0, ty = 0, tx = 0;
    if (tv) {
        const int per_img = g.TH * g.TW;
        n = t / per_img;
        const int r = t - n * per_img;
        ty = r / g.TW;
        tx = r - ty * g.TW;
    }

    // ---- input transform job: (channel cl of the slice, tile tl, half hf of the patch) ----
    // Phase 1 gathers columns 3hf .. 3hf+2 of the 6x6 patch and transforms them (B^T d);
    // phase 2, after the exchange, transforms rows 3hf .. 3hf+2 ((B^T d) B) into V.
    const int cl = (tid >> 5) & (kWfCs - 1);
    const int hf = tid >> 7;
    const int ih0 = 4 * ty - g.PH, iw0 = 4 * tx - g.PW + 3 * hf;
    // Element offsets of the patch rows / columns relative to the patch origin; a
    // row or column outside the image (or past the last tile) gets 2^28, which puts
    // the load past the end of x (x is at most 2^29 bytes), where it reads 0.
    constexpr uint32_t kOut = 1u << 28;
    uint32_t roff[6], coff3[3];
#pragma unroll
    for (int a = 0; a < 6; ++a) roff[a] = (tv && (unsigned)(ih0 + a) < (unsigned)g.H) ? (uint32_t)(a * g.W) : kOut;
#pragma unroll
    for (int b = 0; b < 3; ++b) coff3[b] = (tv && (unsigned)(iw0 + b) < (unsigned)g.W) ? (uint32_t)b : kOut;
    const int hw = g.H * g.W;
    const uint32_t xorg = (uint32_t)(n * g.C * hw + ih0 * g.W + iw0); // channel 0 (mod 2^32)
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, g.x_bytes);
    auto load_half = [&](int s, float (&d)[6][3]) {
        const int c = s * kWfCs + cl;
        const uint32_t base = c < g.C ? xorg + (uint32_t)(c * hw) : kOut;
#pragma unroll
        for (int a = 0; a < 6; ++a)
#pragma unroll
            for (int b = 0; b < 3; ++b) d[a][b] = buf_f32(rx, (base + roff[a] + coff3[b]) * 4u);
    };
    auto columns = [&](const float (&d)[6][3]) {
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            const float col[6] = {d[0][b], d[1][b], d[2][b], d[3][b], d[4][b], d[5][b]};
            float o[6];
            bt6(col, o);
#pragma unroll
            for (int i = 0; i < 6; ++i) xch[((i * 6 + 3 * hf + b) * kWfCs + cl) * kWfT + tl] = o[i];
        }
    };
    auto rows = [&](float *vb) {
#pragma unroll
        for (int ii = 0; ii < 3; ++ii) {
            const int i = 3 * hf + ii;
            float row[6];
#pragma unroll
            for (int j = 0; j < 6; ++j) row[j] = xch[((i * 6 + j) * kWfCs + cl) * kWfT + tl];
            float o[6];
            bt6(row, o);
#pragma unroll
            for (int j = 0; j < 6; ++j) vb[((i * 6 + j) * kWfCs + cl) * kWfT + tl] = o[j];
        }
    };

    // ---- the 36 GEMMs: A = U slice, B = V slice, both from LDS ----
    // U slice element e = (pos, c, oc) = (e / 128, e / 32 % 4, e % 32): thread tid
    // loads e = tid + 256 i (i < 18), U[pos][c0 + c][oc0 + oc] in global memory, or 0
    // past C or OC (an offset of 2^28 elements, past U's at most 2^29 bytes).
    constexpr int kUPer = kWfSlice / 256; // 18
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(U, g.u_bytes);
    const int u_oc = oc0 + (tid & 31);
    const int u_c = (tid >> 5) & (kWfCs - 1);
    const int u_pos = tid >> 7; // + 2 i
    auto load_u = [&](int s, float (&uv)[kUPer]) {
        const int c = s * kWfCs + u_c;
        const uint32_t ub = (c < g.C && u_oc < g.OC) ? (uint32_t)((u_pos * g.C + c) * g.OC + u_oc) : kOut;
        const uint32_t step = (uint32_t)(2 * g.C * g.OC); // two positions
#pragma unroll
        for (int i = 0; i < kUPer; ++i) uv[i] = buf_f32(ru, (ub + (uint32_t)i * step) * 4u);
    };
    auto store_u = [&](const float (&uv)[kUPer]) {
#pragma unroll
        for (int i = 0; i < kUPer; ++i) us[tid + 256 * i] = uv[i];
    };
    const int pos0 = kWfUnits * wave;

    f32x16 acc[kWfUnits];
#pragma unroll
    for (int j = 0; j < kWfUnits; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;

    // Patches are loaded two K slices ahead (register buffers pa / pb in turn): slice s
    // computes from V slice s % 2 while slice s + 1's patches, issued during slice s - 1,
    // are transformed and slice s + 2's are loaded. With fewer workgroups than CUs each
    // workgroup's slices form one chain, and a one-slice distance left every slice
    // waiting out a memory round trip.
    float pa[6][3], pb[6][3];
    float uv[kUPer];
    load_half(0, pa);
    load_u(0, uv);
    if (S > 1) load_half(1, pb);
    columns(pa);
    __syncthreads();
    rows(vs0);
    store_u(uv);
    __syncthreads();
    // dn: slice s + 1's patches (loaded); df: consumed, receives slice s + 2's
    auto slice = [&](int s, const float (&dn)[6][3], float (&df)[6][3]) {
        const float *cur = (s & 1) ? vs1 : vs0;
        float *nxt = (s & 1) ? vs0 : vs1;
        const bool more = s + 1 < S;
        if (more) load_u(s + 1, uv); // in flight during this slice's MFMAs
        if (s + 2 < S) load_half(s + 2, df);
#pragma unroll
        for (int q = 0; q < kWfCs / 2; ++q) {
            const int brow = (2 * q + h) * kWfT + l32;
            float av[kWfUnits], bv[kWfUnits];
#pragma unroll
            for (int j = 0; j < kWfUnits; ++j) {
                av[j] = us[(pos0 + j) * kWfCs * kWfT + brow];
                bv[j] = cur[(pos0 + j) * kWfCs * kWfT + brow];
            }
#pragma unroll
            for (int j = 0; j < kWfUnits; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j], bv[j], acc[j], 0, 0, 0);
        }
        if (more) columns(dn);
        __syncthreads(); // exchange area complete; every wave is past this slice's MFMAs
        if (more) {
            rows(nxt);
            store_u(uv);
        }
        __syncthreads(); // next V and U slices complete, exchange area free
    };
    int s = 0;
    for (; s + 1 < S; s += 2) {
        slice(s, pb, pa);
        slice(s + 1, pa, pb);
    }
    if (s < S) slice(s, pb, pa);

    // ---- output transform: 4 rounds of 8 of the 32 output channels ----
    // Staged layout [position][r % 4][lane half][32 tiles] over both V slices: the two
    // half-waves of a store or a read are 32 words apart (no bank conflicts).
    const int hsel = (tid >> 5) & 1, rr = (tid >> 6) & 3;
    const int row8 = 4 * hsel + rr;
    const int ohw = g.OH * g.OW;
    for (int g4 = 0; g4 < 4; ++g4) {
        if (g4) __syncthreads(); // the previous pass's reads are done
#pragma unroll
        for (int j = 0; j < kWfUnits; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) lds[(((pos0 + j) * 4 + q) * 2 + h) * 32 + l32] = acc[j][4 * g4 + q];
        __syncthreads();
        const int oc = oc0 + 8 * g4 + row8;
        if (!tv || oc >= g.OC) continue;
        const float *mp = lds + (rr * 2 + hsel) * 32 + tl; // position p at mp[p * 256]
        float tc[4][6]; // A^T M: column j -> 4 values
#pragma unroll
        for (int j = 0; j < 6; ++j) {
            float col[6];
#pragma unroll
            for (int i = 0; i < 6; ++i) col[i] = mp[(i * 6 + j) * 256];
            float o[4];
            at6(col, o);
#pragma unroll
            for (int i = 0; i < 4; ++i) tc[i][j] = o[i];
        }
        const float b = bias ? bias[oc] : 0.f;
        const int ybase = (n * g.OC + oc) * ohw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float o[4];
            at6(tc[i], o);
            const int oh = 4 * ty + i;
            if (oh >= g.OH) continue;
            const int row = ybase + oh * g.OW + 4 * tx;
            if (vec_out) {
                float4 v = make_float4(o[0] + b, o[1] + b, o[2] + b, o[3] + b);
                if (res) {
                    const float4 rv = *reinterpret_cast<const float4 *>(res + row);
                    v.x += rv.x;
                    v.y += rv.y;
                    v.z += rv.z;
                    v.w += rv.w;
                }
                v = make_float4(apply_act_c<AC>(v.x), apply_act_c<AC>(v.y), apply_act_c<AC>(v.z),
                                apply_act_c<AC>(v.w));
                *reinterpret_cast<float4 *>(y + row) = v;
            } else {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    if (4 * tx + jj >= g.OW) break;
                    float v = o[jj] + b;
                    if (res) v += res[row + jj];
                    y[row + jj] = apply_act_c<AC>(v);
                }
            }
        }
    }
}

int g_fused_mode = -1; // spinn_hip_tune_winograd_fused: -1 rule, 0 never, 1 whenever eligible

int env_fused() {
    // SPINN_WINOGRAD_FUSED=0 keeps every F(4x4,3x3) layer on the three launches,
    // 1 fuses every eligible one; unset = per-shape choice.
    static int v = [] {
        const char *e = std::getenv("SPINN_WINOGRAD_FUSED");
        if (!e || !*e) return -1;
        return e[0] == '0' ? 0 : 1;
    }();
    return v;
}

void launch_fused(const dim3 &grid, int act, hipStream_t st, const float *x, const float *U, const float *bias,
                  const float *res, float *y, const WfGeom &g, int vec_out) {
    const int ac = act_class(act);
    if (ac == 1)
        hipLaunchKernelGGL((wino4_fused_kernel<1>), grid, dim3(256), 0, st, x, U, bias, res, y, g, vec_out);
    else if (ac == 3)
        hipLaunchKernelGGL((wino4_fused_kernel<3>), grid, dim3(256), 0, st, x, U, bias, res, y, g, vec_out);
    else
        hipLaunchKernelGGL((wino4_fused_kernel<0>), grid, dim3(256), 0, st, x, U, bias, res, y, g, vec_out);
}

} // namespace

void force_winograd_fused(int mode) { g_fused_mode = mode < 0 ? -1 : (mode ? 1 : 0); }

// Shapes the fused kernel can take: 32-bit element offsets for x, y and U.
static bool fused_fits(const SpinnHipConvDesc *d) {
    const int64_t xe = (int64_t)d->n * d->c * d->h * d->w;
    const int64_t ye = (int64_t)d->n * d->oc * d->oh * d->ow;
    const int64_t ue = (int64_t)36 * d->c * d->oc;
    const int64_t tiles = (int64_t)d->n * ((d->oh + 3) / 4) * ((d->ow + 3) / 4);
    // x and U at most 2^29 bytes: an offset past them is formed by adding 2^28 elements
    // (2^30 bytes) to an origin that may sit up to two rows before the image
    return xe * 4 <= (1ll << 29) && ye <= INT32_MAX && ue * 4 <= (1ll << 29) && tiles <= INT32_MAX - kWfT &&
           d->ph <= 2 && d->pw <= 2;
}

bool wino4_fused_selected(const SpinnHipConvDesc *d) {
    if (!winograd_eligible(d) || !fused_fits(d)) return false;
    const int mode = g_fused_mode >= 0 ? g_fused_mode : env_fused();
    if (mode >= 0) return mode == 1;
    // Per-shape rule (measured on MI355X, graph-timed layers): the fused kernel wins
    // where V and M would be large against the GEMM work - at most 64 input channels -
    // and there are enough 32-tile blocks to keep two workgroups on most CUs (a lone
    // workgroup's K slices are latency-bound: 2.7 us each). At batch 32 / 16:
    // 64@56x56 62.7 against 68.8 us (three launches), 64@80x80 65.8 against 69.7,
    // 32@160x160 71.3 against 96.7 (implicit GEMM), 16@160x160 39.9 against 56.8;
    // 128@28x28 87.6 against 49.7 and 128@40x40 82.8 against 48.8 stay on three
    // launches, as do batch-1 layers (64@56x56: 44.6 against 11.5).
    const int64_t tiles = (int64_t)d->n * ((d->oh + 3) / 4) * ((d->ow + 3) / 4);
    return d->c <= 64 && tiles >= 4096;
}

int wino4_fused_conv(const SpinnHipConvDesc *d, const float *x, const float *U, const float *bias,
                     const float *res, float *y, hipStream_t st) {
    if (!fused_fits(d)) return SPINN_HIP_EUNSUPPORTED;
    WfGeom g;
    g.C = d->c;
    g.H = d->h;
    g.W = d->w;
    g.OC = d->oc;
    g.OH = d->oh;
    g.OW = d->ow;
    g.PH = d->ph;
    g.PW = d->pw;
    g.TH = (d->oh + 3) / 4;
    g.TW = (d->ow + 3) / 4;
    g.T = d->n * g.TH * g.TW;
    g.x_bytes = (uint32_t)((int64_t)d->n * d->c * d->h * d->w * 4);
    g.u_bytes = (uint32_t)((int64_t)36 * d->c * d->oc * 4);
    // float4 output rows: whole 4-pixel tile rows and 16-byte aligned y / residual rows
    const int vec_out = (d->ow % 4 == 0 && ((uintptr_t)y & 15u) == 0 && ((uintptr_t)res & 15u) == 0) ? 1 : 0;
    const unsigned bx = (unsigned)((g.T + kWfT - 1) / kWfT);
    launch_fused(dim3(bx, (unsigned)((d->oc + 31) / 32)), d->act, st, x, U, bias, res, y, g, vec_out);
    return check_launch();
}

} // namespace spinn
