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

template <int C, bool RES>
__global__ __launch_bounds__(256) void stem7_mfma_kernel(const float *__restrict__ x, const float *__restrict__ wpk,
                                                         const float *__restrict__ bias, const float *__restrict__ res,
                                                         float *__restrict__ y, SpinnHipConvDesc d, int ldw) {
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
    const uint32_t a_lane0 = l32 < ldw ? (uint32_t)(h * ldw + l32) * 4u : kOOB;
    const uint32_t a_lane1 = l32 + 32 < ldw ? (uint32_t)(h * ldw + l32 + 32) * 4u : kOOB;
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
        const float a1 = buf_f32(rw, a_lane1 + (uint32_t)s * a_step);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b, acc1, 0, 0, 0);
    }
    if (n >= d.ow) return;
    // The bias comes from LDS and every residual load is issued before the first
    // store: one wait per lane instead of a global round trip per output.
    // (acc + bias) + residual, the epilogue's order.
    const int64_t ohw = (int64_t)d.oh * d.ow;
    const int64_t base = (int64_t)img * d.oc * ohw + (int64_t)oh * d.ow + n;
    if constexpr (!RES) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < d.oc) y[base + (int64_t)m * ohw] = apply_act((mb ? acc1[r] : acc0[r]) + bsh[m], d.act);
            }
        return;
    }
    float v[2][16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int mr = 8 * (r >> 2) + 4 * h + (r & 3);
        v[0][r] = acc0[r] + bsh[mr];
        v[1][r] = acc1[r] + bsh[32 + mr];
    }
    {
        float rv[2][16];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                rv[mb][r] = m < d.oc ? res[base + (int64_t)m * ohw] : 0.f;
            }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) v[mb][r] += rv[mb][r];
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m < d.oc) y[base + (int64_t)m * ohw] = apply_act(v[mb][r], d.act);
        }
}

} // namespace

bool stem_mfma_eligible(const SpinnHipConvDesc *d) {
    return d->group == 1 && d->c >= 1 && d->c <= 4 && d->kh == kStemK && d->kw == kStemK && d->sh == kStemS &&
           d->sw == kStemS && d->ph == kStemP && d->pw == kStemP && d->oc >= 1 && d->oc <= kStemOC &&
           d->ow >= 1 && d->ow <= kStemPX && d->oh >= 1 && (int64_t)d->n * d->oh <= INT32_MAX &&
           (int64_t)d->n * d->c * d->h * d->w * 4 <= (int64_t)kMaxOperandBytes;
}

// packed: the implicit GEMM's W^T [K][ldw] with K in (c, kh, kw) order (C < 16).
int stem_mfma_conv(const SpinnHipConvDesc *d, const float *x, const float *packed, const float *bias,
                   const float *res, float *y, hipStream_t st) {
    if (!packed) return SPINN_HIP_EINVAL;
    const int ldw = (d->oc + 3) / 4 * 4;
    const dim3 grid((unsigned)(d->n * d->oh));
    if (res) {
        switch (d->c) {
        case 1: hipLaunchKernelGGL((stem7_mfma_kernel<1, true>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        case 2: hipLaunchKernelGGL((stem7_mfma_kernel<2, true>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        case 3: hipLaunchKernelGGL((stem7_mfma_kernel<3, true>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        default: hipLaunchKernelGGL((stem7_mfma_kernel<4, true>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        }
    } else {
        switch (d->c) {
        case 1: hipLaunchKernelGGL((stem7_mfma_kernel<1, false>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        case 2: hipLaunchKernelGGL((stem7_mfma_kernel<2, false>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        case 3: hipLaunchKernelGGL((stem7_mfma_kernel<3, false>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        default: hipLaunchKernelGGL((stem7_mfma_kernel<4, false>), grid, dim3(256), 0, st, x, packed, bias, res, y, *d, ldw); break;
        }
    }
    return check_launch();
}

} // namespace spinn
