// conv_gemm.hip - implicit-GEMM convolution and Gemm/MatMul on fp32 MFMA.
//
// Convolution as GEMM, SPINN orientation (SPINN/run_time/ops/conv/conv2d.c:184-225):
//   M = OC/g (output channels), N = batch*OH*OW (output pixels, batch folded
//   into N instead of the reference's per-image loop), K = C/g*KH*KW (taps).
// The A operand is the weight matrix re-laid out once as W^T [K][OCg padded to 4]
// (the plan-time counterpart of sgemm_pack_a_offline, gemm_kernel.c:346-369);
// the B operand is never materialised: each K slice of im2col is gathered from
// NCHW input straight into LDS (no column buffer, unlike conv2d.c:172-193).
// The bias / residual / ReLU / SiLU epilogue (gemm_kernel.c:316-338) is fused:
// bias + residual are the accumulators' start value, the activation is applied
// before the only store of the output.
//
// When the tile grid is too small to fill 256 CUs, K is split over blockIdx.z:
// each split writes raw partial sums to the workspace and a reduction kernel
// sums them in a fixed order and applies the epilogue (deterministic).
#include "mfma_core.h"
#include "spinn_hip_internal.h"
#include "streamk.h"
#include <type_traits>

namespace spinn {

struct ConvKArgs {
    const float *wpk;  // packed W^T: [group][K][ldw]
    int64_t wpk_group_stride;
    int ldw;
    int M, K;          // per group
    ConvGeom geom;
    float *__restrict__ y;
    const float *__restrict__ bias;
    const float *__restrict__ res;
    uint32_t res_bytes; // extent of res (the output's size)
    int act;
    int OC, OHW;
    float *__restrict__ ws; // split-K partials [split][OC][ntot]
    int k_chunk;       // K per split (multiple of kBK)
};

// Accumulator start values of a conv output tile: bias + residual when
// `terms` (their loads then overlap the K loop's prologue instead of arriving
// as one burst of reads after it, and the epilogue only applies the activation
// and stores; the sum is the reference's acc + bias + residual in another
// order, within fp32 rounding), else zero.
template <class WT>
__device__ __forceinline__ void conv_acc_start(const ConvKArgs &a, int group, int m0, int n0, int wm0, int wn0,
                                               int lane, bool terms, f32x16 (&c)[WT::TM][WT::TN]) {
    if (!terms) {
        ZeroAcc{}(c);
        return;
    }
    // Unconditional buffer loads: a missing bias or residual is a zero-sized
    // resource and rows or columns past the edge read at kOOB, all of which
    // return 0.
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias ? a.bias + group * a.M : a.y, a.bias ? (uint32_t)a.M * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res ? a.res : a.y, a.res ? a.res_bytes : 0u);
#pragma unroll
    for (int j = 0; j < WT::TN; ++j) {
        const int jcol = n0 + wn0 + j * 32 + l32;
        const bool col_ok = jcol < a.geom.ntot;
        const int img = jcol / a.OHW;
        const int p = jcol - img * a.OHW;
        const uint32_t ybase = ((uint32_t)img * a.OC + (uint32_t)(group * a.M)) * a.OHW + p;
#pragma unroll
        for (int i = 0; i < WT::TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const bool ok = m < a.M;
                const float bv = buf_f32(rb, ok ? (uint32_t)m * 4u : kOOB);
                const float rv = buf_f32(rr, ok && col_ok ? (ybase + (uint32_t)m * a.OHW) * 4u : kOOB);
                c[i][j][r] = bv + rv;
            }
    }
}

// Post-op and store of a finished conv output tile (accumulators already hold
// bias + residual). Lane owns columns n0 + wn0 + j*32 + lane%32 and rows
// m0 + wm0 + i*32 + 8*(r/4) + 4*(lane/32) + r%4.
template <class WT, int AC>
__device__ __forceinline__ void conv_store(const ConvKArgs &a, int group, int m0, int n0, int wm0, int wn0, int lane,
                                           const f32x16 (&acc)[WT::TM][WT::TN]) {
    const int h = lane >> 5;
    const int l32 = lane & 31;
    // A tile whose rows all exist (the usual case: OC a multiple of the tile)
    // stores without a per-element row test.
    const bool full_m = m0 + WT::WM * WT::WAVES_M <= a.M;
#pragma unroll
    for (int j = 0; j < WT::TN; ++j) {
        const int jcol = n0 + wn0 + j * 32 + l32;
        if (jcol >= a.geom.ntot) continue;
        const int img = jcol / a.OHW;
        const int p = jcol - img * a.OHW;
        float *yp = a.y + ((int64_t)img * a.OC + (int64_t)group * a.M + m0 + wm0 + 4 * h) * a.OHW + p;
        if (full_m) {
#pragma unroll
            for (int i = 0; i < WT::TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    yp[(int64_t)(i * 32 + 8 * (r >> 2) + (r & 3)) * a.OHW] = apply_act_c<AC>(acc[i][j][r]);
        } else {
#pragma unroll
            for (int i = 0; i < WT::TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int mo = i * 32 + 8 * (r >> 2) + (r & 3);
                    if (m0 + wm0 + 4 * h + mo < a.M) yp[(int64_t)mo * a.OHW] = apply_act_c<AC>(acc[i][j][r]);
                }
        }
    }
}

// AC: the post-op class (act_class), fixed at compile time so the epilogue has no
// per-element branch on it.
template <int BM, int BN, int BK, class BLoader, bool SPLIT, int AC>
__global__ __launch_bounds__(kThreads, 2) void conv_igemm_kernel(ConvKArgs a) {
    using WT = WaveTiling<BM, BN>;
    constexpr int SA = LdsPad<BM>::stride;
    constexpr int SB = LdsPad<BN>::stride;
    __shared__ __attribute__((aligned(16))) float As[2][BK * SA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = WT::origin_m(wave);
    const int wn0 = WT::origin_n(wave);
    int tile_m, tile_n;
    xcd_tile(gridDim.y, gridDim.x, tile_m, tile_n);
    const int n0 = tile_n * BN;
    const int m0 = tile_m * BM;
    const int z = blockIdx.z;
    const int group = SPLIT ? 0 : z;
    const int k_begin = SPLIT ? z * a.k_chunk : 0;
    const int k_end = SPLIT ? min(a.K, k_begin + a.k_chunk) : a.K;

    KMajorLoader<BM, BK, true> al;
    al.init(a.wpk + group * a.wpk_group_stride, (uint32_t)a.K * (uint32_t)a.ldw * 4u, (uint32_t)a.ldw, m0, a.ldw);
    BLoader bl;
    bl.init(a.geom, n0, group, tid, k_end);

    const int h = lane >> 5;
    const int l32 = lane & 31;
    const int ntot = a.geom.ntot;
    auto init = [&](f32x16 (&c)[WT::TM][WT::TN]) {
        conv_acc_start<WT>(a, group, m0, n0, wm0, wn0, lane, !SPLIT, c);
    };

    f32x16 acc[WT::TM][WT::TN];
    const int nslices = (k_end - k_begin + BK - 1) / BK;
    gemm_mainloop<BM, BN, BK, kStages>(al, bl, As, Bs, acc, k_begin, nslices, tid, lane, wm0, wn0, init);

    if constexpr (SPLIT) {
#pragma unroll
        for (int j = 0; j < WT::TN; ++j) {
            const int jcol = n0 + wn0 + j * 32 + l32;
            if (jcol >= ntot) continue;
            float *wsz = a.ws + (int64_t)z * a.OC * ntot + jcol;
#pragma unroll
            for (int i = 0; i < WT::TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < a.M) wsz[(int64_t)m * ntot] = acc[i][j][r];
                }
        }
    } else {
        conv_store<WT, AC>(a, group, m0, n0, wm0, wn0, lane, acc);
    }
}

// K slices [k0, k1) of output tile t of a group-1 conv into acc, through the
// shared K loop; the accumulators start from bias + residual when k0 == 0.
template <int BM, int BN, int BK, class BLoader>
__device__ __forceinline__ void conv_segment(const ConvKArgs &a, int tiles_m, int t, int k0, int k1,
                                             float (*As)[BK * LdsPad<BM>::stride],
                                             float (*Bs)[BK * LdsPad<BN>::stride],
                                             f32x16 (&acc)[WaveTiling<BM, BN>::TM][WaveTiling<BM, BN>::TN], int tid,
                                             int lane, int wm0, int wn0, int &m0, int &n0) {
    using WT = WaveTiling<BM, BN>;
    m0 = (t % tiles_m) * BM;
    n0 = (t / tiles_m) * BN;
    const int mm0 = m0, nn0 = n0;
    KMajorLoader<BM, BK, true> al;
    al.init(a.wpk, (uint32_t)a.K * (uint32_t)a.ldw * 4u, (uint32_t)a.ldw, m0, a.ldw);
    BLoader bl;
    bl.init(a.geom, n0, 0, tid, min(a.K, k1 * BK));
    auto init = [&](f32x16 (&c)[WT::TM][WT::TN]) { conv_acc_start<WT>(a, 0, mm0, nn0, wm0, wn0, lane, k0 == 0, c); };
    gemm_mainloop<BM, BN, BK, kStages>(al, bl, As, Bs, acc, k0 * BK, k1 - k0, tid, lane, wm0, wn0, init);
}

// Data-parallel + stream-K launch of a group-1 conv (streamk.h). SPLIT_WGS:
// block ids below 8 * s.W run a range of at most S slices of the remaining
// tiles (the end of one tile and the start of the next), the rest one whole
// tile each. PARTS_IN_DP: every block runs one whole tile, the first R * p of
// them a part of a remaining tile before it. Segments are unrolled: a loop
// would keep the second segment's set-up live across the first segment's K
// loop and cost a wave per SIMD.
template <int BM, int BN, int BK, class BLoader, int AC, int SCHEME>
__global__ __launch_bounds__(kThreads, 2) void conv_igemm_sk_kernel(ConvKArgs a, SkSched s) {
    using WT = WaveTiling<BM, BN>;
    constexpr int SA = LdsPad<BM>::stride;
    constexpr int SB = LdsPad<BN>::stride;
    constexpr int NA = WT::TM * WT::TN * 16; // accumulators per thread
    constexpr int TILE = BM * BN;            // floats of one partial tile
    __shared__ __attribute__((aligned(16))) float As[2][BK * SA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];
    __shared__ int sk_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = WT::origin_m(wave);
    const int wn0 = WT::origin_n(wave);
    const int id = blockIdx.x;
    const int nsk = SCHEME == kSkSplitWgs ? kXcds * s.W : 0;
    const int x = (id < nsk ? id : id - nsk) % kXcds;
    int xstart, count;
    sk_xcd_tiles(s, x, xstart, count);
    const int tile_sk0 = kXcds * s.dp_per_xcd + xstart; // this XCD's first remaining tile
    int m0, n0;

    if (SCHEME == kSkSplitWgs && id < nsk) {
        // SPLIT_WGS: one range of the XCD's remaining slices
        const int I = count * s.S;
        const int Wx = min(s.W, I);
        const int w = id / kXcds;
        if (w >= Wx) return; // no slices for this workgroup (uniform exit)
        const int b = sk_begin(w, I, Wx);
        const int e = sk_begin(w + 1, I, Wx);
#pragma unroll
        for (int seg = 0; seg < 2; ++seg) {
            const int i = seg == 0 ? b : (b / s.S + 1) * s.S;
            if (i >= e) break;
            const int r = i / s.S;
            const int k0 = i - r * s.S;
            const int k1 = min(s.S, k0 + (e - i));
            f32x16 acc[WT::TM][WT::TN];
            conv_segment<BM, BN, BK, BLoader>(a, s.tiles_m, tile_sk0 + r, k0, k1, As, Bs, acc, tid, lane, wm0, wn0,
                                              m0, n0);
            if (k0 == 0 && k1 == s.S) {
                conv_store<WT, AC>(a, 0, m0, n0, wm0, wn0, lane, acc);
            } else {
                const int w_first = sk_owner(r * s.S, I, Wx);
                const int nparts = sk_owner((r + 1) * s.S - 1, I, Wx) - w_first + 1;
                f32x16 sum[WT::TM][WT::TN];
                auto slot_of = [&](int q) {
                    const int wq = w_first + q;
                    return (x * s.W + wq) * 2 + ((sk_begin(wq, I, Wx) / s.S == r) ? 0 : 1);
                };
                if (sk_finish_part<NA, TILE>(s, kXcds * s.W * 2, (x * s.W + w) * 2 + seg, xstart + r, nparts,
                                             reinterpret_cast<const float *>(&acc), reinterpret_cast<float *>(&sum),
                                             tid, sk_last, slot_of))
                    conv_store<WT, AC>(a, 0, m0, n0, wm0, wn0, lane, sum);
            }
            __syncthreads(); // the next segment's prologue rewrites the LDS buffers
        }
        return;
    }

    const int l = (id - nsk) / kXcds; // XCD-local index of this whole-tile workgroup
    if (SCHEME == kSkPartsInDp && l < count * s.p) {
        // PARTS_IN_DP: part j of remaining tile r first
        const int r = l / s.p;
        const int j = l - r * s.p;
        const int k0 = j * s.S / s.p;
        const int k1 = (j + 1) * s.S / s.p;
        f32x16 acc[WT::TM][WT::TN];
        conv_segment<BM, BN, BK, BLoader>(a, s.tiles_m, tile_sk0 + r, k0, k1, As, Bs, acc, tid, lane, wm0, wn0, m0,
                                          n0);
        f32x16 sum[WT::TM][WT::TN];
        const int base = (x * s.rx + r) * s.p;
        auto slot_of = [&](int q) { return base + q; };
        if (sk_finish_part<NA, TILE>(s, kXcds * s.rx * s.p, base + j, xstart + r, s.p,
                                     reinterpret_cast<const float *>(&acc), reinterpret_cast<float *>(&sum), tid,
                                     sk_last, slot_of))
            conv_store<WT, AC>(a, 0, m0, n0, wm0, wn0, lane, sum);
        __syncthreads(); // the whole tile's prologue rewrites the LDS buffers
    }
    f32x16 acc[WT::TM][WT::TN];
    conv_segment<BM, BN, BK, BLoader>(a, s.tiles_m, x * s.dp_per_xcd + l, 0, s.S, As, Bs, acc, tid, lane, wm0, wn0,
                                      m0, n0);
    conv_store<WT, AC>(a, 0, m0, n0, wm0, wn0, lane, acc);
}

// Sum split-K partials in split order and apply the conv epilogue.
__global__ __launch_bounds__(256) void conv_splitk_reduce_kernel(const float *__restrict__ ws, int nsplit,
                                                                 int OC, int ntot, int OHW,
                                                                 const float *__restrict__ bias,
                                                                 const float *__restrict__ res, int act,
                                                                 float *__restrict__ y) {
    const int64_t total = (int64_t)OC * ntot;
    const int64_t plane = total;
    const bool narrow = total <= INT32_MAX; // 32-bit index division (uniform branch)
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int oc = narrow ? (int)((uint32_t)e / (uint32_t)ntot) : (int)(e / ntot);
        const int jcol = (int)(e - (int64_t)oc * ntot);
        float v = splitk_sum(ws, nsplit, plane, e);
        const int img = jcol / OHW;
        const int p = jcol - img * OHW;
        const int64_t idx = ((int64_t)img * OC + oc) * OHW + p;
        if (bias) v += bias[oc];
        if (res) v += res[idx];
        y[idx] = apply_act(v, act);
    }
}

// W [group][OCg][Cg][KH][KW] -> W^T [group][K][ldw], K in tap-major (kh,kw,c)
// order when tap_order, else (c,kh,kw); columns OCg..ldw-1 are zero.
__global__ void conv_pack_wt_kernel(const float *__restrict__ w, float *__restrict__ out, int groups, int OCg,
                                    int Cg, int KHW, int ldw, int tap_order) {
    const int K = Cg * KHW;
    const int64_t total = (int64_t)groups * K * ldw;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int m = (int)(e % ldw);
        const int64_t gk = e / ldw;
        const int k = (int)(gk % K);
        const int g = (int)(gk / K);
        float v = 0.f;
        if (m < OCg) {
            int c, tap;
            if (tap_order) {
                tap = k / Cg;
                c = k - tap * Cg;
            } else {
                c = k / KHW;
                tap = k - c * KHW;
            }
            v = w[(((int64_t)g * OCg + m) * Cg + c) * KHW + tap];
        }
        out[e] = v;
    }
}

// W [OC][Cg][KH][KW] -> [OC][K] with K in tap-major (kh, kw, c) order.
__global__ void conv_pack_kcopy_kernel(const float *__restrict__ w, float *__restrict__ out, int OC, int Cg,
                                       int KHW) {
    const int K = Cg * KHW;
    const int64_t total = (int64_t)OC * K;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int k = (int)(e % K);
        const int64_t oc = e / K;
        const int tap = k / Cg;
        const int c = k - tap * Cg;
        out[e] = w[(oc * Cg + c) * KHW + tap];
    }
}

// ---------------------------------------------------------------------------
// Host side: tile selection and launch.
// ---------------------------------------------------------------------------
namespace {

template <int BM, int BN, class BL>
int launch_conv_tile(const ConvKArgs &a, int groups, int split, hipStream_t st) {
    dim3 grid((a.geom.ntot + BN - 1) / BN, (a.M + BM - 1) / BM, split > 1 ? split : groups);
    if (split > 1) // the post-op runs in the reduction kernel
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, kBK, BL, true, 0>), grid, dim3(kThreads), 0, st, a);
    else if (act_class(a.act) == 1)
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, kBK, BL, false, 1>), grid, dim3(kThreads), 0, st, a);
    else if (act_class(a.act) == 3)
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, kBK, BL, false, 3>), grid, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, kBK, BL, false, 0>), grid, dim3(kThreads), 0, st, a);
    return check_launch();
}

template <int BM, int BN, class BL>
int launch_conv_sk_tile(const ConvKArgs &a, const SkPlan &sp, int S, void *ws, hipStream_t st) {
    SkSched s{};
    s.tiles_m = (a.M + BM - 1) / BM;
    s.S = S;
    s.dp_per_xcd = sp.dp_per_xcd;
    s.R = sp.R;
    s.scheme = sp.scheme;
    s.W = sp.W;
    s.p = sp.p;
    s.rx = (sp.R + kXcds - 1) / kXcds;
    s.local = xcd_local_parts() ? 1 : 0;
    s.epoch = streamk_epoch();
    s.cnt = (unsigned long long *)ws;
    s.part = (float *)((char *)ws + sp.cnt_bytes);
    s.status = device_status_word();
    s.tries = streamk_tries();
    const dim3 grid(sp.grid);
    if (sp.scheme == kSkSplitWgs) {
        if (act_class(a.act) == 1)
            hipLaunchKernelGGL((conv_igemm_sk_kernel<BM, BN, kBK, BL, 1, kSkSplitWgs>), grid, dim3(kThreads), 0, st,
                               a, s);
        else if (act_class(a.act) == 3)
            hipLaunchKernelGGL((conv_igemm_sk_kernel<BM, BN, kBK, BL, 3, kSkSplitWgs>), grid, dim3(kThreads), 0, st,
                               a, s);
        else
            hipLaunchKernelGGL((conv_igemm_sk_kernel<BM, BN, kBK, BL, 0, kSkSplitWgs>), grid, dim3(kThreads), 0, st,
                               a, s);
    } else {
        if (act_class(a.act) == 1)
            hipLaunchKernelGGL((conv_igemm_sk_kernel<BM, BN, kBK, BL, 1, kSkPartsInDp>), grid, dim3(kThreads), 0, st,
                               a, s);
        else if (act_class(a.act) == 3)
            hipLaunchKernelGGL((conv_igemm_sk_kernel<BM, BN, kBK, BL, 3, kSkPartsInDp>), grid, dim3(kThreads), 0, st,
                               a, s);
        else
            hipLaunchKernelGGL((conv_igemm_sk_kernel<BM, BN, kBK, BL, 0, kSkPartsInDp>), grid, dim3(kThreads), 0, st,
                               a, s);
    }
    return check_launch();
}

template <template <int> class BLT>
int launch_conv_sk(const ConvKArgs &a, const TileChoice &tc, const SkPlan &sp, int S, void *ws, hipStream_t st) {
    if (tc.bm == 32 && tc.bn == 128) return launch_conv_sk_tile<32, 128, BLT<128>>(a, sp, S, ws, st);
    if (tc.bm == 128 && tc.bn == 128) return launch_conv_sk_tile<128, 128, BLT<128>>(a, sp, S, ws, st);
    if (tc.bm == 128 && tc.bn == 64) return launch_conv_sk_tile<128, 64, BLT<64>>(a, sp, S, ws, st);
    if (tc.bm == 64 && tc.bn == 128) return launch_conv_sk_tile<64, 128, BLT<128>>(a, sp, S, ws, st);
    return launch_conv_sk_tile<64, 64, BLT<64>>(a, sp, S, ws, st);
}

template <template <int> class BLT>
int launch_conv_bl(const ConvKArgs &a, const TileChoice &tc, int groups, hipStream_t st) {
    if (tc.bm == 128 && tc.bn == 128) return launch_conv_tile<128, 128, BLT<128>>(a, groups, tc.split, st);
    if (tc.bm == 128 && tc.bn == 64) return launch_conv_tile<128, 64, BLT<64>>(a, groups, tc.split, st);
    if (tc.bm == 64 && tc.bn == 128) return launch_conv_tile<64, 128, BLT<128>>(a, groups, tc.split, st);
    if (tc.bm == 32 && tc.bn == 128) return launch_conv_tile<32, 128, BLT<128>>(a, groups, tc.split, st);
    return launch_conv_tile<64, 64, BLT<64>>(a, groups, tc.split, st);
}

template <int BN> using TapBL = Im2colTapLoader<BN, kBK>;
template <int BN> using Gen33BL = Im2colLoader<BN, kBK, 3, 3>;
template <int BN> using Gen77BL = Im2colLoader<BN, kBK, 7, 7>;
template <int BN> using Gen11BL = Im2colLoader<BN, kBK, 1, 1>;
template <int BN> using GenBL = Im2colLoader<BN, kBK, 0, 0>;

template <int BN> using PwBL = Pointwise1x1Loader<BN, kBK>;

bool conv_tap_order(const SpinnHipConvDesc *d) { return ((d->c / d->group) % kBK) == 0; }

// 1x1 / stride 1 / no padding over planes of a multiple of 4 pixels, 16-byte
// aligned input: the B operand is read as float4 runs of the input itself.
bool conv_pointwise_vec(const SpinnHipConvDesc *d, const float *x) {
    return d->kh == 1 && d->kw == 1 && d->sh == 1 && d->sw == 1 && d->ph == 0 && d->pw == 0 && d->oh == d->h &&
           d->ow == d->w && (d->oh * d->ow) % 4 == 0 && ((uintptr_t)x & 15u) == 0;
}

} // namespace

// Floats of the W^T section [group][K][ldw] of the packed weights.
static int64_t igemm_wt_floats(const SpinnHipConvDesc *d) {
    const int OCg = d->oc / d->group;
    const int ldw = (OCg + 3) / 4 * 4;
    const int64_t K = (int64_t)(d->c / d->group) * d->kh * d->kw;
    return (int64_t)d->group * K * ldw;
}

// Tap-ordered windows larger than 1x1 also keep W with K contiguous, [group][OCg][K]
// in the same tap order, after W^T: the wave-K kernel's A operand then moves four k
// per 16-byte load, as it does from the raw weights of a 1x1 conv.
static bool igemm_has_kcopy(const SpinnHipConvDesc *d) { return conv_tap_order(d) && d->kh * d->kw > 1; }

int64_t igemm_packed_floats(const SpinnHipConvDesc *d) {
    const int64_t K = (int64_t)(d->c / d->group) * d->kh * d->kw;
    return igemm_wt_floats(d) + (igemm_has_kcopy(d) ? (int64_t)d->oc * K : 0);
}

const float *igemm_kcopy(const SpinnHipConvDesc *d, const float *packed) {
    return (packed && igemm_has_kcopy(d)) ? packed + igemm_wt_floats(d) : nullptr;
}

int igemm_pack(const SpinnHipConvDesc *d, const float *w, float *packed, hipStream_t st) {
    const int OCg = d->oc / d->group;
    const int ldw = (OCg + 3) / 4 * 4;
    const int64_t total = igemm_wt_floats(d);
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 65535);
    hipLaunchKernelGGL(conv_pack_wt_kernel, dim3(blocks), dim3(256), 0, st, w, packed, d->group, OCg,
                       d->c / d->group, d->kh * d->kw, ldw, conv_tap_order(d) ? 1 : 0);
    int rc = check_launch();
    if (rc || !igemm_has_kcopy(d)) return rc;
    const int64_t kc = (int64_t)d->oc * (d->c / d->group) * d->kh * d->kw;
    const int kblocks = (int)std::min<int64_t>((kc + 255) / 256, 65535);
    hipLaunchKernelGGL(conv_pack_kcopy_kernel, dim3(kblocks), dim3(256), 0, st, w, packed + total, d->oc,
                       d->c / d->group, d->kh * d->kw);
    return check_launch();
}

static TileChoice igemm_tiles(const SpinnHipConvDesc *d) {
    const int OCg = d->oc / d->group;
    const int K = (d->c / d->group) * d->kh * d->kw;
    const int ntot = d->n * d->oh * d->ow;
    return choose_tiles(OCg, ntot, K, d->group, d->group == 1);
}

// Data-parallel + stream-K split for a group-1 conv whose tile count leaves
// the CUs unevenly loaded (any tile shape).
static bool igemm_streamk(const SpinnHipConvDesc *d, const TileChoice &tc, SkPlan &sp) {
    // A grid the tile rule already splits along K (long K, few tiles) keeps its
    // split: several workgroups per CU hide the gather latency better than one
    // or two whole tiles and an extra range.
    if (d->group != 1 || tc.split > 1) return false;
    const int K = d->c * d->kh * d->kw;
    const int ntot = d->n * d->oh * d->ow;
    return plan_streamk((d->oc + tc.bm - 1) / tc.bm, (ntot + tc.bn - 1) / tc.bn, (K + kBK - 1) / kBK,
                        tc.bm * tc.bn, sp);
}

static int igemm_wavek(const SpinnHipConvDesc *d) {
    const bool pointwise = d->kh == 1 && d->kw == 1 && d->sh == 1 && d->sw == 1 && d->ph == 0 && d->pw == 0 &&
                           d->oh == d->h && d->ow == d->w;
    return wavek_tile(d->oc / d->group, d->n * d->oh * d->ow, (d->c / d->group) * d->kh * d->kw, d->group,
                      pointwise ? kWkConvPointwise : kWkConvGather);
}

static bool igemm_stem(const SpinnHipConvDesc *d) { return stem_mfma_eligible(d) && !tiles_forced(); }

size_t igemm_workspace_bytes(const SpinnHipConvDesc *d) {
    if (igemm_stem(d) || igemm_wavek(d)) return 0;
    TileChoice tc = igemm_tiles(d);
    SkPlan sp;
    if (igemm_streamk(d, tc, sp)) {
        // plan time: settle how the parts exchange sums on this device
        int dev = 0;
        if (hipGetDevice(&dev) == hipSuccess) probe_xcd_local(dev);
        init_device_status();
        return sp.ws_bytes;
    }
    if (tc.split <= 1) return 0;
    return (size_t)tc.split * d->oc * ((size_t)d->n * d->oh * d->ow) * sizeof(float);
}

int igemm_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed, const float *bias,
               const float *res, float *y, void *ws, size_t ws_bytes, hipStream_t st) {
    if (igemm_stem(d)) return stem_mfma_conv(d, x, packed, bias, res, y, st);
    if (const int ts = igemm_wavek(d)) return wavek_conv(d, ts, x, w, packed, bias, res, y, st);
    ConvKArgs a{};
    const int OCg = d->oc / d->group;
    a.ldw = (OCg + 3) / 4 * 4;
    a.M = OCg;
    a.K = (d->c / d->group) * d->kh * d->kw;
    a.wpk = packed;
    a.wpk_group_stride = (int64_t)a.K * a.ldw;
    const uint64_t x_bytes = (uint64_t)d->n * d->c * d->h * d->w * sizeof(float);
    const uint64_t w_bytes = (uint64_t)igemm_wt_floats(d) * sizeof(float);
    const uint64_t y_bytes = (uint64_t)d->n * d->oc * d->oh * d->ow * sizeof(float);
    if (x_bytes > kMaxOperandBytes || w_bytes > kMaxOperandBytes || y_bytes > kMaxOperandBytes)
        return SPINN_HIP_EUNSUPPORTED;
    a.geom = ConvGeom{x, (uint32_t)x_bytes, d->c, d->h, d->w, d->c / d->group, d->oh, d->ow, d->kh, d->kw,
                      d->sh, d->sw, d->ph, d->pw, d->n * d->oh * d->ow};
    a.y = y;
    a.bias = bias;
    a.res = res;
    a.res_bytes = (uint32_t)y_bytes;
    a.act = d->act;
    a.OC = d->oc;
    a.OHW = d->oh * d->ow;
    TileChoice tc = igemm_tiles(d);
    SkPlan sp;
    if (igemm_streamk(d, tc, sp)) {
        if (!ws || ws_bytes < sp.ws_bytes || ((uintptr_t)ws & 15u)) return SPINN_HIP_EWORKSPACE;
        const int S = (a.K + kBK - 1) / kBK;
        if (conv_pointwise_vec(d, x)) return launch_conv_sk<PwBL>(a, tc, sp, S, ws, st);
        if (conv_tap_order(d)) return launch_conv_sk<TapBL>(a, tc, sp, S, ws, st);
        if (d->kh == 3 && d->kw == 3) return launch_conv_sk<Gen33BL>(a, tc, sp, S, ws, st);
        if (d->kh == 7 && d->kw == 7) return launch_conv_sk<Gen77BL>(a, tc, sp, S, ws, st);
        if (d->kh == 1 && d->kw == 1) return launch_conv_sk<Gen11BL>(a, tc, sp, S, ws, st);
        return launch_conv_sk<GenBL>(a, tc, sp, S, ws, st);
    }
    if (tc.split > 1) {
        const size_t need = (size_t)tc.split * d->oc * (size_t)a.geom.ntot * sizeof(float);
        if (!ws || ws_bytes < need) return SPINN_HIP_EWORKSPACE;
        a.ws = (float *)ws;
        a.k_chunk = tc.k_chunk;
    }
    int rc;
    if (conv_pointwise_vec(d, x)) rc = launch_conv_bl<PwBL>(a, tc, d->group, st);
    else if (conv_tap_order(d)) rc = launch_conv_bl<TapBL>(a, tc, d->group, st);
    else if (d->kh == 3 && d->kw == 3) rc = launch_conv_bl<Gen33BL>(a, tc, d->group, st);
    else if (d->kh == 7 && d->kw == 7) rc = launch_conv_bl<Gen77BL>(a, tc, d->group, st);
    else if (d->kh == 1 && d->kw == 1) rc = launch_conv_bl<Gen11BL>(a, tc, d->group, st);
    else rc = launch_conv_bl<GenBL>(a, tc, d->group, st);
    if (rc) return rc;
    if (tc.split > 1) {
        const int64_t total = (int64_t)d->oc * a.geom.ntot;
        const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
        hipLaunchKernelGGL(conv_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, (const float *)ws,
                           tc.split, d->oc, a.geom.ntot, a.OHW, bias, res, d->act, y);
        rc = check_launch();
    }
    return rc;
}

} // namespace spinn
