// glue.hip - bandwidth kernels around the conv/GEMM path: MaxPool2d,
// mean reduction (ReduceMean / GlobalAveragePool) and a 32-bit fill.
#include "mfma_core.h"
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

// Pools with a K/2 pad over 16-byte input rows and output rows of at most 256
// pixels (3x3 stride 1 or 2, 5x5 stride 1: ResNet's stem pool, YOLO's SPPF):
// one wave per (plane, run of bands of RB output rows), lanes over 4-pixel
// quads of the row, each input row of a band one 16-byte load per lane (two at
// stride 2), the K/2 neighbour columns from the adjacent lanes by a lane
// permute. Taps outside the image read -inf, which never beats the running
// maximum's start of -1e30: the same result as skipping them. Taps are taken
// in the reference's (kh, kw) order with its `v > m` rule, so NaN is never
// selected and the result is bit-identical to the per-output kernels above.
template <int K, int S, int RB>
__global__ __launch_bounds__(256) void maxpool_wave_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                           SpinnHipPoolDesc d, int owq, int bands, int bpw, int wpp,
                                                           int waves) {
    constexpr int HL = S == 1 ? K / 2 : 1;
    constexpr int HR = S == 1 ? K / 2 : 0;
    constexpr int NV = HL + 4 * S + HR;
    constexpr int IR = (RB - 1) * S + K;
    const float ninf = -__builtin_inff();
    const int lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t pl = wave / (uint32_t)wpp;
    const int bg = (int)(wave - pl * (uint32_t)wpp);
    const int bl = lane / owq, q = lane - bl * owq;
    const int b = bg * bpw + bl;
    const bool on = wave < (uint32_t)waves && bl < bpw && b < bands;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(((int64_t)d.n * d.c) * d.h * d.w * 4));
    const uint32_t plane_off = pl * (uint32_t)(d.h * d.w);
    const int ih0 = b * RB * S - d.ph;
    const int col0 = 4 * S * q;
    const bool has_l = q > 0, has_r = q + 1 < owq;
    const int addr_l = (lane - 1) << 2, addr_r = (lane + 1) << 2;
    f32x4 f[IR][S];
    bool rok[IR];
#pragma unroll
    for (int ir = 0; ir < IR; ++ir) {
        const int ih = ih0 + ir;
        rok[ir] = on && (unsigned)ih < (unsigned)d.h;
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int col = col0 + 4 * u;
            const bool ok = rok[ir] && col < d.w;
            f[ir][u] = buf_f32x4(rx, ok ? (plane_off + (uint32_t)ih * d.w + col) * 4u : kOOB);
            if (!ok) f[ir][u] = f32x4{ninf, ninf, ninf, ninf};
        }
    }
    float m[RB][4];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) m[r][j] = -1e30f;
#pragma unroll
    for (int ir = 0; ir < IR; ++ir) {
        float v[NV];
#pragma unroll
        for (int u = 0; u < S; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[HL + 4 * u + e] = f[ir][u][e];
#pragma unroll
        for (int j = 0; j < HL; ++j) {
            const float t =
                __int_as_float(__builtin_amdgcn_ds_bpermute(addr_l, __float_as_int(f[ir][S - 1][4 - HL + j])));
            v[j] = has_l ? t : ninf;
        }
#pragma unroll
        for (int j = 0; j < HR; ++j) {
            const float t = __int_as_float(__builtin_amdgcn_ds_bpermute(addr_r, __float_as_int(f[ir][0][j])));
            v[HL + 4 * S + j] = has_r ? t : ninf;
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int kh = ir - r * S;
            if (kh >= 0 && kh < K) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int kw = 0; kw < K; ++kw) {
                        const float t = v[j * S + kw];
                        m[r][j] = t > m[r][j] ? t : m[r][j];
                    }
            }
        }
    }
    if (!on) return;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int oh = b * RB + r;
        if (oh >= d.oh) break;
        const int ow0 = 4 * q;
        const int64_t o = ((int64_t)pl * d.oh + oh) * d.ow + ow0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (ow0 + j < d.ow) y[o + j] = m[r][j];
    }
}

template <int K, int S, int RB>
static int launch_maxpool_wave(const SpinnHipPoolDesc *d, const float *x, float *y, hipStream_t st) {
    const int owq = (d->ow + 3) / 4;
    const int bands = (d->oh + RB - 1) / RB;
    const int bpw = 64 / owq;
    const int wpp = (bands + bpw - 1) / bpw;
    const int64_t waves = (int64_t)d->n * d->c * wpp;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks * 256 > INT32_MAX) return SPINN_HIP_EUNSUPPORTED;
    hipLaunchKernelGGL((maxpool_wave_kernel<K, S, RB>), dim3((unsigned)blocks), dim3(256), 0, st, x, y, *d, owq,
                       bands, bpw, wpp, (int)waves);
    return check_launch();
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

// inner == 1 with rows of at most kMeanRowMax floats (GlobalAveragePool over a
// 7x7 map): a one-wave workgroup stages 64 consecutive rows in LDS - one
// contiguous run, moved with 16-byte loads all issued before the first LDS
// store - then each lane sums its row in order from 0, as the reference's loop
// does (SPINN/run_time/ops/reduce/reduce_mean.c:68-72), so the result is
// bit-identical to it. Rows sit at an odd float stride in LDS (the row length
// itself when odd, so the staging store needs no division; even rows get one
// float of padding): the lanes read distinct banks.
constexpr int kMeanRowMax = 63;
constexpr int kMeanRows = 64;
constexpr int kMeanVec = (kMeanRows * kMeanRowMax / 4 + 63) / 64; // 16-byte loads per lane, at most
template <bool ODD> // ODD: stride == dim
__global__ __launch_bounds__(64) void mean_rows_lds_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                           int64_t rows, int dim, int stride) {
    __shared__ float rowbuf[kMeanRows * kMeanRowMax];
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kMeanRows;
    const int nr = (int)min<int64_t>(kMeanRows, rows - r0);
    const int n = nr * dim;
    const float *xb = x + r0 * dim;
    const int nv = n >> 2;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xb, (uint32_t)n * 4u);
    f32x4 q[kMeanVec];
#pragma unroll
    for (int i = 0; i < kMeanVec; ++i) {
        const int v = lane + 64 * i;
        q[i] = buf_f32x4(rx, v < nv ? (uint32_t)v * 16u : kOOB);
    }
    const int et = 4 * nv + lane; // tail: n % 4 < 4 floats
    const float t = et < n ? xb[et] : 0.f;
#pragma unroll
    for (int i = 0; i < kMeanVec; ++i) {
        const int v = lane + 64 * i;
        if (v < nv) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = 4 * v + u;
                rowbuf[ODD ? e : e + e / dim] = q[i][u];
            }
        }
    }
    if (et < n) rowbuf[ODD ? et : et + et / dim] = t;
    __syncthreads();
    if (lane >= nr) return;
    const float *rp = rowbuf + lane * stride;
    float s = 0.f;
    for (int j = 0; j < dim; ++j) s += rp[j];
    y[r0 + lane] = s / (float)dim;
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
    const bool wave_ok = d->kh == d->kw && d->sh == d->sw && d->ph == d->kh / 2 && d->pw == d->kw / 2 &&
                         d->w % 4 == 0 && d->ow <= 256 && d->ow == (d->w + 2 * d->pw - d->kw) / d->sw + 1 &&
                         d->oh == (d->h + 2 * d->ph - d->kh) / d->sh + 1 && (int64_t)planes * d->h * d->w * 4 <= (int64_t)kMaxOperandBytes;
    if (wave_ok && d->kh == 3 && d->sh == 1) return launch_maxpool_wave<3, 1, 2>(d, x, y, st);
    if (wave_ok && d->kh == 3 && d->sh == 2) return launch_maxpool_wave<3, 2, 1>(d, x, y, st);
    if (wave_ok && d->kh == 5 && d->sh == 1) return launch_maxpool_wave<5, 1, 2>(d, x, y, st);
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
    if (inner == 1 && dim <= kMeanRowMax && ((uintptr_t)x & 15) == 0) {
        const int stride = (int)dim | 1;
        const int64_t blocks = (outer + kMeanRows - 1) / kMeanRows;
        if (blocks <= INT32_MAX) {
            if (dim & 1)
                hipLaunchKernelGGL(mean_rows_lds_kernel<true>, dim3((unsigned)blocks), dim3(64), 0, st, x, y, outer,
                                   (int)dim, stride);
            else
                hipLaunchKernelGGL(mean_rows_lds_kernel<false>, dim3((unsigned)blocks), dim3(64), 0, st, x, y, outer,
                                   (int)dim, stride);
            return check_launch();
        }
    }
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
