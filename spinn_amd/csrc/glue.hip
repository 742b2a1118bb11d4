// glue.hip - bandwidth kernels around the conv/GEMM path: MaxPool2d,
// mean reduction (ReduceMean / GlobalAveragePool) and a 32-bit fill.
#include "spinn_hip_internal.h"

namespace spinn {

// One thread per output element, ow fastest (SPINN/run_time/ops/pool/maxpool.c:28-46:
// window taps outside the input are skipped; an empty window yields -1e30).
__global__ __launch_bounds__(256) void maxpool_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                      SpinnHipPoolDesc d) {
    const int64_t total = (int64_t)d.n * d.c * d.oh * d.ow;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int ow = (int)(e % d.ow);
        const int64_t t = e / d.ow;
        const int oh = (int)(t % d.oh);
        const int64_t nc = t / d.oh;
        const float *xp = x + nc * d.h * d.w;
        float m = -1e30f;
        for (int kh = 0; kh < d.kh; ++kh) {
            const int ih = oh * d.sh - d.ph + kh;
            if ((unsigned)ih >= (unsigned)d.h) continue;
            for (int kw = 0; kw < d.kw; ++kw) {
                const int iw = ow * d.sw - d.pw + kw;
                if ((unsigned)iw >= (unsigned)d.w) continue;
                const float v = xp[(int64_t)ih * d.w + iw];
                m = v > m ? v : m;
            }
        }
        y[e] = m;
    }
}

// The same pooling with the plane on grid.y (a stride of gridDim.y over the
// planes) and one thread per output pixel of the plane on grid.x: 32-bit index
// math instead of the 64-bit divisions of a flat output index (ResNet-101's
// 3x3/2 pool at batch 32: 49 us before).
__global__ __launch_bounds__(256) void maxpool_plane_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                            SpinnHipPoolDesc d, int planes) {
    const int ohw = d.oh * d.ow;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= ohw) return;
    const int oh = p / d.ow;
    const int ow = p - oh * d.ow;
    const int ih0 = oh * d.sh - d.ph, iw0 = ow * d.sw - d.pw;
    const int hw = d.h * d.w;
    for (int pl = blockIdx.y; pl < planes; pl += gridDim.y) {
        const float *xp = x + (int64_t)pl * hw;
        float m = -1e30f;
        for (int kh = 0; kh < d.kh; ++kh) {
            const int ih = ih0 + kh;
            if ((unsigned)ih >= (unsigned)d.h) continue;
            for (int kw = 0; kw < d.kw; ++kw) {
                const int iw = iw0 + kw;
                if ((unsigned)iw >= (unsigned)d.w) continue;
                const float v = xp[ih * d.w + iw];
                m = v > m ? v : m;
            }
        }
        y[(int64_t)pl * ohw + p] = m;
    }
}

// inner == 1: one wave per output, lanes stride the reduced axis, then a
// wave-shuffle tree (SPINN/run_time/ops/reduce/reduce_mean.c:68-74).
__global__ __launch_bounds__(256) void mean_rows_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                        int64_t rows, int64_t dim) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t r = wave; r < rows; r += nwaves) {
        const float *xp = x + r * dim;
        float s = 0.f;
        for (int64_t i = lane; i < dim; i += 64) s += xp[i];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) y[r] = s / (float)dim;
    }
}

// inner > 1: one thread per (outer, inner), consecutive threads on inner.
__global__ __launch_bounds__(256) void mean_strided_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                           int64_t outer, int64_t dim, int64_t inner) {
    const int64_t total = outer * inner;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t o = e / inner;
        const int64_t k = e - o * inner;
        const float *xp = x + o * dim * inner + k;
        float s = 0.f;
        for (int64_t j = 0; j < dim; ++j) s += xp[j * inner];
        y[e] = s / (float)dim;
    }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *__restrict__ p, uint32_t v, int64_t n) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x)
        p[e] = v;
}

static int grid_for(int64_t n, int per_block = 256, int cap = 16384) {
    return (int)std::max<int64_t>(1, std::min<int64_t>((n + per_block - 1) / per_block, cap));
}

int maxpool2d(const SpinnHipPoolDesc *d, const float *x, float *y, hipStream_t st) {
    const int64_t total = (int64_t)d->n * d->c * d->oh * d->ow;
    if (total == 0) return 0;
    const int64_t planes = (int64_t)d->n * d->c;
    if ((int64_t)d->h * d->w <= INT32_MAX && (int64_t)d->oh * d->ow <= INT32_MAX - 256 && planes <= INT32_MAX) {
        const dim3 grid((unsigned)((d->oh * d->ow + 255) / 256), (unsigned)std::min<int64_t>(planes, 65535));
        hipLaunchKernelGGL(maxpool_plane_kernel, grid, dim3(256), 0, st, x, y, *d, (int)planes);
    } else {
        hipLaunchKernelGGL(maxpool_kernel, dim3(grid_for(total)), dim3(256), 0, st, x, y, *d);
    }
    return check_launch();
}

int reduce_mean(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, hipStream_t st) {
    if (outer * inner == 0) return 0;
    if (inner == 1) {
        hipLaunchKernelGGL(mean_rows_kernel, dim3(grid_for(outer * 64)), dim3(256), 0, st, x, y, outer, dim);
    } else {
        hipLaunchKernelGGL(mean_strided_kernel, dim3(grid_for(outer * inner)), dim3(256), 0, st, x, y, outer, dim,
                           inner);
    }
    return check_launch();
}

int fill_u32(void *dst, uint32_t value, size_t bytes, hipStream_t st) {
    const int64_t n = (int64_t)(bytes / 4);
    if (n == 0) return 0;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n)), dim3(256), 0, st, (uint32_t *)dst, value, n);
    return check_launch();
}

} // namespace spinn
