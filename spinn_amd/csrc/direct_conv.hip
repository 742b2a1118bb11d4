// direct_conv.hip - grouped / depthwise convolution as a bandwidth kernel.
//
// The reference runs these through its per-group im2col + GEMM loop
// (SPINN/run_time/ops/conv/conv2d.c:178-227), which for depthwise is an M=1
// axpy per channel (SPINN/run_time/ops/mm/gemm_kernel.c:215-241) followed by
// the epilogue (:316-338). Depthwise work is a few flops per byte, so this
// kernel is organised for HBM: one thread per output pixel, consecutive
// threads on consecutive ow (coalesced loads and stores), the channel's
// KHxKW filter broadcast from scalar registers, the epilogue fused.
#include "spinn_hip_internal.h"

namespace spinn {

// grid.x: tiles of 256 output pixels of one (n, oc) plane; grid.y: n*OC planes.
template <int KH, int KW>
__global__ __launch_bounds__(256) void direct_conv_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                          const float *__restrict__ bias,
                                                          const float *__restrict__ res, float *__restrict__ y,
                                                          SpinnHipConvDesc d) {
    const int kh_n = KH > 0 ? KH : d.kh;
    const int kw_n = KW > 0 ? KW : d.kw;
    const int plane = blockIdx.y; // n*OC + oc
    const int n = plane / d.oc;
    const int oc = plane - n * d.oc;
    const int ohw = d.oh * d.ow;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= ohw) return;
    const int oh = p / d.ow;
    const int ow = p - oh * d.ow;
    const int OCg = d.oc / d.group;
    const int Cg = d.c / d.group;
    const int g = oc / OCg;
    const int ih0 = oh * d.sh - d.ph;
    const int iw0 = ow * d.sw - d.pw;
    const float *wp = w + (int64_t)oc * Cg * kh_n * kw_n;
    float acc = 0.f;
    for (int c = 0; c < Cg; ++c) {
        const float *xp = x + ((int64_t)n * d.c + (int64_t)g * Cg + c) * d.h * d.w;
        const float *wc = wp + c * kh_n * kw_n;
        for (int kh = 0; kh < kh_n; ++kh) {
            const int ih = ih0 + kh;
            if ((unsigned)ih >= (unsigned)d.h) continue;
            for (int kw = 0; kw < kw_n; ++kw) {
                const int iw = iw0 + kw;
                if ((unsigned)iw < (unsigned)d.w) acc = fmaf(wc[kh * kw_n + kw], xp[(int64_t)ih * d.w + iw], acc);
            }
        }
    }
    const int64_t idx = (int64_t)plane * ohw + p;
    float v = acc;
    if (bias) v += bias[oc];
    if (res) v += res[idx];
    y[idx] = apply_act(v, d.act);
}

int direct_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias, const float *res,
                float *y, hipStream_t st) {
    const int ohw = d->oh * d->ow;
    const int64_t planes = (int64_t)d->n * d->oc;
    if (planes > 2147483647LL) return SPINN_HIP_EUNSUPPORTED;
    dim3 grid((ohw + 255) / 256, (unsigned)planes);
    if (d->kh == 3 && d->kw == 3)
        hipLaunchKernelGGL((direct_conv_kernel<3, 3>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
    else if (d->kh == 5 && d->kw == 5)
        hipLaunchKernelGGL((direct_conv_kernel<5, 5>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
    else if (d->kh == 7 && d->kw == 7)
        hipLaunchKernelGGL((direct_conv_kernel<7, 7>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
    else
        hipLaunchKernelGGL((direct_conv_kernel<0, 0>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
    return check_launch();
}

} // namespace spinn
