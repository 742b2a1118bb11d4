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

    // Lane owns columns jcol = n0 + wn0 + j*32 + lane%32 and rows
    // m0 + wm0 + i*32 + 8*(r/4) + 4*(lane/32) + r%4 of the tile.
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const int ntot = a.geom.ntot;

    // Without split K the accumulators start from the epilogue's additive
    // terms, bias + residual: their loads then overlap the K loop's prologue
    // instead of arriving as one burst of reads after it, and the epilogue
    // only applies the activation and stores. (The sum is the reference's
    // acc + bias + residual in another order, within fp32 rounding.)
    auto init = [&](f32x16 (&c)[WT::TM][WT::TN]) {
        if constexpr (SPLIT) {
            ZeroAcc{}(c);
        } else {
            // Unconditional buffer loads: a missing bias or residual is a
            // zero-sized resource and rows or columns past the edge read at
            // kOOB, all of which return 0.
            const __amdgpu_buffer_rsrc_t rb =
                make_rsrc(a.bias ? a.bias + group * a.M : a.y, a.bias ? (uint32_t)a.M * 4u : 0u);
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res ? a.res : a.y, a.res ? a.res_bytes : 0u);
#pragma unroll
            for (int j = 0; j < WT::TN; ++j) {
                const int jcol = n0 + wn0 + j * 32 + l32;
                const bool col_ok = jcol < ntot;
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
        // A tile whose rows all exist (the usual case: OC a multiple of the tile)
        // stores without a per-element row test.
        const bool full_m = m0 + BM <= a.M;
#pragma unroll
        for (int j = 0; j < WT::TN; ++j) {
            const int jcol = n0 + wn0 + j * 32 + l32;
            if (jcol >= ntot) continue;
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

static int igemm_wavek(const SpinnHipConvDesc *d) {
    const bool pointwise = d->kh == 1 && d->kw == 1 && d->sh == 1 && d->sw == 1 && d->ph == 0 && d->pw == 0 &&
                           d->oh == d->h && d->ow == d->w;
    return wavek_tile(d->oc / d->group, d->n * d->oh * d->ow, (d->c / d->group) * d->kh * d->kw, d->group,
                      pointwise);
}

size_t igemm_workspace_bytes(const SpinnHipConvDesc *d) {
    if (igemm_wavek(d)) return 0;
    TileChoice tc = igemm_tiles(d);
    if (tc.split <= 1) return 0;
    return (size_t)tc.split * d->oc * ((size_t)d->n * d->oh * d->ow) * sizeof(float);
}

int igemm_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed, const float *bias,
               const float *res, float *y, void *ws, size_t ws_bytes, hipStream_t st) {
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
