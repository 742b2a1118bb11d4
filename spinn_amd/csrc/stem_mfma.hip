// stem_mfma.hip - the 7x7 stride-2 stem convolution of an image network (up to
// 4 input channels, up to 64 output channels, output rows of up to 128
// pixels: ResNet's 3 -> 64 stem at 224x224) as an MFMA kernel over an
// LDS-staged input window.
//
// One workgroup computes one output row: all output channels x the row's
// pixels. It stages the row's input window - C channels x 7 input rows x
// (2 * 128 + 6) columns, zero outside the image (the conv padding) - in LDS
// once, then runs the whole K range (K = C*49 in the reference's (c, kh, kw)
// im2col order, SPINN/run_time/ops/conv/conv2d.c:58-76) as a fully unrolled
// chain of v_mfma_f32_32x32x2f32 steps whose B operands are LDS reads at
// compile-time offsets and whose A operands come from the packed weights
// W^T [K][ldw] through the caches. The generic implicit GEMM
// decodes (c, kh, kw) for every element of every K slice and gathers it from
// global memory; here the im2col is an address constant. Each wave owns 32 of
// the row's pixels and both 32-channel blocks; bias, residual and the post-op
// are applied on the way out (SPINN/run_time/ops/mm/gemm_kernel.c:316-338).
// With SPLIT (grids of fewer rows than CUs: batch 1 and 2 at 224x224) two
// workgroups share a row, blockIdx.y choosing the 32-channel block: twice the
// workgroups, each with half the MFMA chain (same steps per output, same bits).
#include "mfma_core.h"
#include "spinn_hip_internal.h"

namespace spinn {

namespace {

constexpr int kStemK = 7, kStemS = 2, kStemP = 3;
constexpr int kStemOC = 64;                       // output channels of the tile (all of them)
constexpr int kStemPX = 128;                      // pixels per output row, at most: 4 waves x 32
constexpr int kStemPW = kStemS * kStemPX + kStemK - 1; // 262 patch columns; column 0 is input column -3

// LDS offset (floats) of input element k = (c, kh, kw) for pixel 0 of the row.
__host__ __device__ constexpr int stem_koff(int k) {
    return ((k / (kStemK * kStemK)) * kStemK + (k % (kStemK * kStemK)) / kStemK) * kStemPW + k % kStemK;
}

template <int C, bool RES, bool SPLIT>
__global__ __launch_bounds__(256) void stem7_mfma_kernel(const float *__restrict__ x, const float *__restrict__ wpk,
                                                         const float *__restrict__ bias, const float *__restrict__ res,
                                                         float *__restrict__ y, SpinnHipConvDesc d, int ldw) {
    constexpr int NMB = SPLIT ? 1 : 2;           // 32-channel blocks this workgroup computes
    const int mb0 = SPLIT ? (int)blockIdx.y : 0; // the first of them
    constexpr int K = C * kStemK * kStemK;
    constexpr int STEPS = (K + 1) / 2; // lane group h supplies k = 2s + h
    __shared__ float patch[C * kStemK * kStemPW]; // [c][kh][col]
    __shared__ float bsh[kStemOC];                // bias, 0 past OC or without one
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int row = blockIdx.x; // img * OH + oh
    const int img = row / d.oh;
    const int oh = row - img * d.oh;
    // Input window of the row's 7 input rows, zero outside the image, staged
    // through registers: every load is issued before the first LDS store.
    constexpr int PN = C * kStemK * kStemPW;
    constexpr int PIT = (PN + 255) / 256;
    const int ih0 = oh * kStemS - kStemP;
    const uint32_t img_off = (uint32_t)img * (uint32_t)(C * d.h * d.w);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)d.n * C * d.h * d.w * 4));
    float pv[PIT];
#pragma unroll
    for (int i = 0; i < PIT; ++i) {
        const int e = tid + i * 256;
        const int rr = e / kStemPW; // c * 7 + kh
        const int col = e - rr * kStemPW;
        const int c = rr / kStemK, kh = rr - c * kStemK;
        const int ih = ih0 + kh, iw = col - kStemP;
        const bool ok = e < PN && (unsigned)ih < (unsigned)d.h && (unsigned)iw < (unsigned)d.w;
        pv[i] = buf_f32(rx, ok ? (img_off + (uint32_t)(c * d.h + ih) * d.w + iw) * 4u : kOOB);
    }
#pragma unroll
    for (int i = 0; i < PIT; ++i) {
        const int e = tid + i * 256;
        if (e < PN) patch[e] = pv[i];
    }
    // A operand straight from the packing W^T [K][ldw] (the same 38 KB for every
    // workgroup: L1 / L2 hits): lane (m = l32 + 32 mb, h) reads row k = 2s + h;
    // rows past K and columns past ldw read 0 through the descriptor's extent.
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wpk, (uint32_t)(K * ldw * 4));
    const int ma = l32 + 32 * mb0;
    const uint32_t a_lane0 = ma < ldw ? (uint32_t)(h * ldw + ma) * 4u : kOOB;
    const uint32_t a_lane1 = ma + 32 < ldw ? (uint32_t)(h * ldw + ma + 32) * 4u : kOOB;
    const uint32_t a_step = (uint32_t)(2 * ldw) * 4u;
    if (tid < kStemOC) bsh[tid] = (bias && tid < d.oc) ? bias[tid] : 0.f;
    __syncthreads();
    const int n = wave * 32 + l32;        // this lane's pixel of the row
    const float *pb = patch + kStemS * n; // B[k][n] = pb[stem_koff(k)]
    f32x16 acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.f;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        // past K (odd K) the weight reads 0 and the B read repeats k = 2s, a finite value
        const int off0 = stem_koff(2 * s);
        const int off1 = 2 * s + 1 < K ? stem_koff(2 * s + 1) : off0;
        const float b = pb[h ? off1 : off0];
        const float a0 = buf_f32(rw, a_lane0 + (uint32_t)s * a_step);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b, acc0, 0, 0, 0);
        if constexpr (!SPLIT) {
            const float a1 = buf_f32(rw, a_lane1 + (uint32_t)s * a_step);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b, acc1, 0, 0, 0);
        }
    }
    if (n >= d.ow) return;
    // The bias comes from LDS and every residual load is issued before the first
    // store: one wait per lane instead of a global round trip per output.
    // (acc + bias) + residual, the epilogue's order.
    const int64_t ohw = (int64_t)d.oh * d.ow;
    const int64_t base = (int64_t)img * d.oc * ohw + (int64_t)oh * d.ow + n;
    if constexpr (!RES) {
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = (mb0 + mb) * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < d.oc) y[base + (int64_t)m * ohw] = apply_act((mb ? acc1[r] : acc0[r]) + bsh[m], d.act);
            }
        return;
    }
    float v[NMB][16];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = (mb0 + mb) * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            v[mb][r] = (mb ? acc1[r] : acc0[r]) + bsh[m];
        }
    {
        float rv[NMB][16];
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = (mb0 + mb) * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                rv[mb][r] = m < d.oc ? res[base + (int64_t)m * ohw] : 0.f;
            }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) v[mb][r] += rv[mb][r];
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = (mb0 + mb) * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m < d.oc) y[base + (int64_t)m * ohw] = apply_act(v[mb][r], d.act);
        }
}


// ---- 3x3 stride-2 stems on v_mfma_f32_16x16x4f32 ----
// Up to 4 input channels, up to 16 output channels, output rows of up to 320
// pixels (YOLOv10n's 3 -> 16 stem at 640x640), begin pads 0 or 1; raw weights
// W [OC][K], K = C*9 in the reference's (c, kh, kw) im2col order
// (SPINN/run_time/ops/conv/conv2d.c:58-76). One workgroup computes one output
// row, all output channels x the row's pixels, from the row's 3 input rows
// staged in LDS (zero outside the image); staged column iw + pw holds input
// column iw, so output pixel ow reads columns 2*ow + kw. 16x16x4 MFMA register
// layout: A lane l = W[oc = l%16][k = 4s + l/16], B lane l = patch[k][pixel l%16],
// accumulator r of lane l = D[oc = 4*(l/16) + r][pixel l%16]: the 16 output
// channels fill the tile's rows exactly, where a 32-row MFMA would leave half
// of them empty. A wave takes every fourth 16-pixel block of the row; its A
// operands (7 steps for 3 channels) and B offsets stay in registers.
constexpr int kS3OC = 16;
constexpr int kS3PX = 320;            // output pixels per row, at most
constexpr int kS3PW = 2 * kS3PX + 2;  // staged columns per input row

template <int C, bool RES>
__global__ __launch_bounds__(256) void stem3_mfma_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                         const float *__restrict__ bias, const float *__restrict__ res,
                                                         float *__restrict__ y, SpinnHipConvDesc d) {
    constexpr int K = C * 9;
    constexpr int STEPS = (K + 3) / 4;
    constexpr int PN = C * 3 * kS3PW;
    constexpr int PIT = (PN + 255) / 256;
    __shared__ float patch[PN]; // [c][kh][col]
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int row = blockIdx.x; // img * OH + oh
    const int img = row / d.oh;
    const int oh = row - img * d.oh;
    const int ih0 = 2 * oh - d.ph;
    // Input rows, every load issued before the first LDS store.
    const uint32_t img_off = (uint32_t)img * (uint32_t)(C * d.h * d.w);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)d.n * C * d.h * d.w * 4));
    float pv[PIT];
#pragma unroll
    for (int i = 0; i < PIT; ++i) {
        const int e = tid + i * 256;
        const int rr = e / kS3PW; // c * 3 + kh
        const int col = e - rr * kS3PW;
        const int c = rr / 3, kh = rr - 3 * c;
        const int ih = ih0 + kh, iw = col - d.pw;
        const bool ok = e < PN && (unsigned)ih < (unsigned)d.h && (unsigned)iw < (unsigned)d.w;
        pv[i] = buf_f32(rx, ok ? (img_off + (uint32_t)(c * d.h + ih) * d.w + iw) * 4u : kOOB);
    }
    // A operands and B offsets of the K steps: k = 4s + g; past K the weight is 0
    // and the B offset points at a staged (finite) value
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(d.oc * K * 4));
    float a[STEPS];
    int boff[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const int k = 4 * s + g;
        const bool ok = k < K;
        a[s] = buf_f32(rw, ok && j < d.oc ? (uint32_t)(j * K + k) * 4u : kOOB);
        const int c = k / 9, kh = (k - 9 * c) / 3, kw = k - 9 * c - 3 * kh;
        boff[s] = ok ? (c * 3 + kh) * kS3PW + kw : 0;
    }
    float bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = (bias && 4 * g + q < d.oc) ? bias[4 * g + q] : 0.f;
#pragma unroll
    for (int i = 0; i < PIT; ++i) {
        const int e = tid + i * 256;
        if (e < PN) patch[e] = pv[i];
    }
    __syncthreads();
    const int64_t ohw = (int64_t)d.oh * d.ow;
    const int nblk = (d.ow + 15) >> 4;
    for (int pb = wave; pb < nblk; pb += 4) {
        const int ow = pb * 16 + j;
        const float *pp = patch + 2 * ow; // ow < 320: columns up to 2*319 + 2 < kS3PW
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < STEPS; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], pp[boff[s]], acc, 0, 0, 0);
        if (ow >= d.ow) continue;
        const int64_t base = (int64_t)img * d.oc * ohw + (int64_t)oh * d.ow + ow;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc[q] + bv[q]; // (acc + bias) + residual, the epilogue's order
        if constexpr (RES) {
            float rv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) rv[q] = 4 * g + q < d.oc ? res[base + (int64_t)(4 * g + q) * ohw] : 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += rv[q];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (4 * g + q < d.oc) y[base + (int64_t)(4 * g + q) * ohw] = apply_act(v[q], d.act);
    }
}

} // namespace

bool stem_mfma_eligible(const SpinnHipConvDesc *d) {
    return d->group == 1 && d->c >= 1 && d->c <= 4 && d->kh == kStemK && d->kw == kStemK && d->sh == kStemS &&
           d->sw == kStemS && d->ph == kStemP && d->pw == kStemP && d->oc >= 1 && d->oc <= kStemOC &&
           d->ow >= 1 && d->ow <= kStemPX && d->oh >= 1 && (int64_t)d->n * d->oh <= INT32_MAX &&
           (int64_t)d->n * d->c * d->h * d->w * 4 <= (int64_t)kMaxOperandBytes;
}

template <int C, bool RES>
static void launch_stem7(const SpinnHipConvDesc *d, const float *x, const float *packed, const float *bias,
                         const float *res, float *y, int ldw, bool split, hipStream_t st) {
    const unsigned rows = (unsigned)(d->n * d->oh);
    if (split)
        hipLaunchKernelGGL((stem7_mfma_kernel<C, RES, true>), dim3(rows, 2), dim3(256), 0, st, x, packed, bias, res, y,
                           *d, ldw);
    else
        hipLaunchKernelGGL((stem7_mfma_kernel<C, RES, false>), dim3(rows), dim3(256), 0, st, x, packed, bias, res, y,
                           *d, ldw);
}

template <bool RES>
static void launch_stem7_c(const SpinnHipConvDesc *d, const float *x, const float *packed, const float *bias,
                           const float *res, float *y, int ldw, bool split, hipStream_t st) {
    switch (d->c) {
    case 1: launch_stem7<1, RES>(d, x, packed, bias, res, y, ldw, split, st); break;
    case 2: launch_stem7<2, RES>(d, x, packed, bias, res, y, ldw, split, st); break;
    case 3: launch_stem7<3, RES>(d, x, packed, bias, res, y, ldw, split, st); break;
    default: launch_stem7<4, RES>(d, x, packed, bias, res, y, ldw, split, st); break;
    }
}

// packed: the implicit GEMM's W^T [K][ldw] with K in (c, kh, kw) order (C < 16).
// Grids of fewer rows than CUs split each row's two 32-channel blocks over two
// workgroups (ResNet-101's stem at batch 1: 112 rows, 14.3 us on one workgroup
// per row).
int stem_mfma_conv(const SpinnHipConvDesc *d, const float *x, const float *packed, const float *bias,
                   const float *res, float *y, hipStream_t st) {
    if (!packed) return SPINN_HIP_EINVAL;
    const int ldw = (d->oc + 3) / 4 * 4;
    const bool split = d->oc > 32 && (int64_t)d->n * d->oh < (int64_t)device_cu_count();
    if (res) launch_stem7_c<true>(d, x, packed, bias, res, y, ldw, split, st);
    else launch_stem7_c<false>(d, x, packed, bias, res, y, ldw, split, st);
    return check_launch();
}

template <int C>
static int launch_stem3(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias,
                        const float *res, float *y, hipStream_t st) {
    const dim3 grid((unsigned)(d->n * d->oh));
    if (res)
        hipLaunchKernelGGL((stem3_mfma_kernel<C, true>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
    else
        hipLaunchKernelGGL((stem3_mfma_kernel<C, false>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
    return check_launch();
}

bool stem3_mfma_eligible(const SpinnHipConvDesc *d) {
    return d->group == 1 && d->c >= 1 && d->c <= 4 && d->kh == 3 && d->kw == 3 && d->sh == 2 && d->sw == 2 &&
           d->ph >= 0 && d->ph <= 1 && d->pw >= 0 && d->pw <= 1 && d->oc >= 1 && d->oc <= kS3OC && d->ow >= 1 &&
           d->ow <= kS3PX && d->oh >= 1 && (int64_t)d->n * d->oh <= INT32_MAX &&
           (int64_t)d->n * d->c * d->h * d->w * 4 <= (int64_t)kMaxOperandBytes;
}

// w: the raw weights W [OC][C][3][3].
int stem3_mfma_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias, const float *res,
                    float *y, hipStream_t st) {
    if (!stem3_mfma_eligible(d)) return SPINN_HIP_EUNSUPPORTED;
    switch (d->c) {
    case 1: return launch_stem3<1>(d, x, w, bias, res, y, st);
    case 2: return launch_stem3<2>(d, x, w, bias, res, y, st);
    case 3: return launch_stem3<3>(d, x, w, bias, res, y, st);
    default: return launch_stem3<4>(d, x, w, bias, res, y, st);
    }
}

} // namespace spinn
