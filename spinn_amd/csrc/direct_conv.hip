// direct_conv.hip - grouped / depthwise convolution as a bandwidth kernel.
//
// The reference runs these through its per-group im2col + GEMM loop
// (SPINN/run_time/ops/conv/conv2d.c:178-227), which for depthwise is an M=1
// axpy per channel (SPINN/run_time/ops/mm/gemm_kernel.c:215-241) followed by
// the epilogue (:316-338). Depthwise work is a few flops per byte, so this
// kernel is organised for HBM: one thread per output pixel, consecutive
// threads on consecutive ow (coalesced loads and stores), the channel's
// KHxKW filter broadcast from scalar registers, the epilogue fused.
#include "mfma_core.h"
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

// Depthwise (one input and one output channel per group): a 32 x 32 tile of
// output pixels per block, its input window (with halo, zero-filled outside the
// image) staged once in LDS, so each input element is read from HBM once per
// tile instead of KH*KW times through the cache. Each thread computes a
// column strip of 4 outputs, reusing every LDS value it reads for all the
// outputs whose window covers it.
constexpr int kDwTH = 32, kDwTW = 32, kDwRows = 4;

template <int K, int S, bool PF>
__global__ __launch_bounds__(256) void dw_tiled_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                       const float *__restrict__ bias, const float *__restrict__ res,
                                                       float *__restrict__ y, SpinnHipConvDesc d, int tiles_w,
                                                       int64_t planes) {
    constexpr int IH = (kDwTH - 1) * S + K; // input rows of a tile
    constexpr int IW = (kDwTW - 1) * S + K; // input cols of a tile
    constexpr int LW = IW + 1;
    constexpr int RIN = (kDwRows - 1) * S + K; // input rows one strip reads
    __shared__ float tile[IH * LW];
    const int tx = threadIdx.x & (kDwTW - 1), ty = threadIdx.x / kDwTW; // ty in [0, 8)
    const int th = blockIdx.x / tiles_w, tw = blockIdx.x - th * tiles_w;
    const int oh0 = th * kDwTH + ty * kDwRows, ow = tw * kDwTW + tx;
    const int ih0 = th * kDwTH * S - d.ph, iw0 = tw * kDwTW * S - d.pw;
    const int64_t hw = (int64_t)d.h * d.w, ohw = (int64_t)d.oh * d.ow;
    // PF (planes of >= 4 tiles, several planes per workgroup): the window of the workgroup's
    // next plane is loaded into registers while this one is computed and stored.
    constexpr int NE = (IH * IW + 255) / 256;
    float v[PF ? NE : 1];
    auto load_window = [&](int64_t pl) {
        const float *xp = x + pl * hw;
#pragma unroll
        for (int u = 0; u < NE; ++u) {
            const int e = threadIdx.x + u * 256;
            const int r = e / IW, q = e - r * IW;
            const int ih = ih0 + r, iw = iw0 + q;
            v[u] = (e < IH * IW && (unsigned)ih < (unsigned)d.h && (unsigned)iw < (unsigned)d.w)
                       ? xp[(int64_t)ih * d.w + iw]
                       : 0.f;
        }
    };
    if constexpr (PF) {
        if ((int64_t)blockIdx.y < planes) load_window(blockIdx.y);
    }
    for (int64_t plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const int c = (int)(plane % d.c);
        if constexpr (PF) {
#pragma unroll
            for (int u = 0; u < NE; ++u) {
                const int e = threadIdx.x + u * 256;
                const int r = e / IW, q = e - r * IW;
                if (e < IH * IW) tile[r * LW + q] = v[u];
            }
        } else {
            const float *xp = x + plane * hw;
            for (int e = threadIdx.x; e < IH * IW; e += 256) {
                const int r = e / IW, q = e - r * IW;
                const int ih = ih0 + r, iw = iw0 + q;
                tile[r * LW + q] = ((unsigned)ih < (unsigned)d.h && (unsigned)iw < (unsigned)d.w)
                                       ? xp[(int64_t)ih * d.w + iw]
                                       : 0.f;
            }
        }
        float wk[K * K];
#pragma unroll
        for (int i = 0; i < K * K; ++i) wk[i] = w[(int64_t)c * K * K + i];
        __syncthreads();
        if constexpr (PF) {
            if (plane + gridDim.y < planes) load_window(plane + gridDim.y);
        }
        float acc[kDwRows];
#pragma unroll
        for (int r = 0; r < kDwRows; ++r) acc[r] = 0.f;
        const float *trow = tile + (ty * kDwRows * S) * LW + tx * S;
#pragma unroll
        for (int ir = 0; ir < RIN; ++ir) {
#pragma unroll
            for (int kw = 0; kw < K; ++kw) {
                const float v = trow[ir * LW + kw];
#pragma unroll
                for (int r = 0; r < kDwRows; ++r) {
                    const int kh = ir - r * S;
                    if (kh >= 0 && kh < K) acc[r] = fmaf(wk[kh * K + kw], v, acc[r]);
                }
            }
        }
        if (ow < d.ow) {
            const float b = bias ? bias[c] : 0.f;
#pragma unroll
            for (int r = 0; r < kDwRows; ++r) {
                const int oh = oh0 + r;
                if (oh < d.oh) {
                    const int64_t idx = plane * ohw + (int64_t)oh * d.ow + ow;
                    float v = acc[r] + b;
                    if (res) v += res[idx];
                    y[idx] = apply_act(v, d.act);
                }
            }
        }
        __syncthreads();
    }
}

// Depthwise convolution without LDS: one thread computes RPT x 4 outputs (RPT
// rows of 4 horizontally adjacent outputs) of one plane, reading each input
// row of its window as three 16-byte loads through a bounds-checked buffer
// (zero outside the image) that the L1 / L2 share between neighbouring
// threads. Thousands of independent threads with a dozen loads each keep the
// HBM queue full without staging; the epilogue is fused and stores float4.
// Needs 16-byte input rows (W % 4 == 0) and the begin column pad K/2 (the
// window's columns then sit at compile-time positions of the three loads).
template <int K, int S, int RPT, bool VEC>
__global__ __launch_bounds__(256) void dw_direct_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                        const float *__restrict__ bias,
                                                        const float *__restrict__ res, float *__restrict__ y,
                                                        SpinnHipConvDesc d, int row_groups, int owq, int64_t total) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    const int64_t per_plane = (int64_t)row_groups * owq;
    const int64_t pl = t / per_plane;
    const int rem = (int)(t - pl * per_plane);
    const int rg = rem / owq;
    const int q = rem - rg * owq;
    const int c = (int)(pl % d.c);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(((int64_t)d.n * d.c) * d.h * d.w * 4));
    float wk[K * K];
#pragma unroll
    for (int i = 0; i < K * K; ++i) wk[i] = w[(int64_t)c * K * K + i];
    constexpr int IR = (RPT - 1) * S + K; // input rows of the thread's window
    const int ih0 = rg * RPT * S - d.ph;
    const int col0 = 4 * q * S - 4; // first column of the three 16-byte loads
    const uint32_t plane_off = (uint32_t)(pl * d.h * d.w);
    float acc[RPT][4];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[r][j] = 0.f;
#pragma unroll
    for (int ir = 0; ir < IR; ++ir) {
        const int ih = ih0 + ir;
        const bool row_ok = (unsigned)ih < (unsigned)d.h;
        float v[12];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int col = col0 + 4 * u;
            const bool ok = row_ok && col >= 0 && col < d.w;
            const f32x4 f = buf_f32x4(rx, ok ? (plane_off + (uint32_t)ih * d.w + col) * 4u : kOOB);
            v[4 * u + 0] = f[0];
            v[4 * u + 1] = f[1];
            v[4 * u + 2] = f[2];
            v[4 * u + 3] = f[3];
        }
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const int kh = ir - r * S;
            if (kh >= 0 && kh < K) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int kw = 0; kw < K; ++kw)
                        acc[r][j] = fmaf(wk[kh * K + kw], v[4 - K / 2 + j * S + kw], acc[r][j]);
            }
        }
    }
    const float bv = bias ? bias[c] : 0.f;
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int oh = rg * RPT + r;
        if (oh >= d.oh) break;
        const int ow0 = 4 * q;
        const int64_t o = (pl * d.oh + oh) * (int64_t)d.ow + ow0;
        if constexpr (VEC) {
            float4 rv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (res) rv = *reinterpret_cast<const float4 *>(res + o);
            float4 out;
            out.x = apply_act(acc[r][0] + bv + rv.x, d.act);
            out.y = apply_act(acc[r][1] + bv + rv.y, d.act);
            out.z = apply_act(acc[r][2] + bv + rv.z, d.act);
            out.w = apply_act(acc[r][3] + bv + rv.w, d.act);
            *reinterpret_cast<float4 *>(y + o) = out;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (ow0 + j < d.ow) {
                    float vv = acc[r][j] + bv;
                    if (res) vv += res[o + j];
                    y[o + j] = apply_act(vv, d.act);
                }
            }
        }
    }
}

// Depthwise convolution, one wave per (plane, run of row bands). The wave's
// lanes split each output row of its plane into 4-pixel quads (owq lanes per
// band) and take bpw = 64 / owq bands of RB output rows each, so the plane's
// filter and bias are wave-uniform and sit in scalar registers. Each input row
// of a band is one 16-byte load per lane (two for stride 2); the K/2 columns
// on either side of a lane's quad are the neighbouring lanes' values, moved by
// a lane permute (zero at the band's ends: the image edge, where the pad is
// K/2). Every wave issues all its loads at once (the filter's scalar loads
// beside them), computes and stores: short bands, many waves (measured on
// YOLOv10n's batch-16 layers: 2- and 3-row bands beat 4- and 8-row ones, and
// beat waves that loop over several bands with the next band's loads in
// flight). Epilogue fused, float4 stores.
constexpr int kDwWaveThreads = 256; // 4 waves per workgroup

template <int K, int S, int RB, bool VEC>
__global__ __launch_bounds__(kDwWaveThreads) void dw_wave_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ bias, const float *__restrict__ res,
                                                      float *__restrict__ y, SpinnHipConvDesc d, int owq, int bands,
                                                      int bpw, int wpp, int waves) {
    static_assert(S == 1 || (S == 2 && K == 3), "stride 2 only for 3 x 3 filters");
    constexpr int HL = S == 1 ? K / 2 : 1; // columns from the left neighbour
    constexpr int HR = S == 1 ? K / 2 : 0; // columns from the right neighbour
    constexpr int NV = HL + 4 * S + HR;     // window columns of one input row
    constexpr int IR = (RB - 1) * S + K;    // input rows of a band
    const int lane = threadIdx.x & 63;
    // the scalar arguments fetched in one round trip before any use
    uint64_t px = (uint64_t)x, pr = (uint64_t)res, py = (uint64_t)y;
    asm volatile(""
                 : "+s"(owq), "+s"(bands), "+s"(bpw), "+s"(wpp), "+s"(waves), "+s"(d.n), "+s"(d.c), "+s"(d.h),
                   "+s"(d.w), "+s"(d.oh), "+s"(d.ow), "+s"(d.ph), "+s"(d.act), "+s"(px), "+s"(pr), "+s"(py));
    typedef __attribute__((address_space(1))) const float gcf;
    typedef __attribute__((address_space(1))) float gf;
    x = (const float *)(gcf *)px;
    res = (const float *)(gcf *)pr;
    y = (float *)(gf *)py;
    // 32-bit index math (the host keeps waves * 64 below 2^31); the waves past
    // the last one of the grid's final workgroup run with every lane off, so
    // no branch holds back the first loads.
    const uint32_t wave =
        blockIdx.x * (uint32_t)(kDwWaveThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t pl = wave / (uint32_t)wpp;
    const int bg = (int)(wave - pl * (uint32_t)wpp);
    const int c = (int)(pl % (uint32_t)d.c);
    const int bl = lane / owq, q = lane - bl * owq;
    const int b = bg * bpw + bl;
    const bool on = wave < (uint32_t)waves && bl < bpw && b < bands;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(((int64_t)d.n * d.c) * d.h * d.w * 4));
    const uint32_t plane_off = pl * (uint32_t)(d.h * d.w);
    const int ih0 = b * RB * S - d.ph;
    const int col0 = 4 * S * q;
    const bool has_l = q > 0, has_r = q + 1 < owq; // neighbour lane in the same band
    const int addr_l = (lane - 1) << 2, addr_r = (lane + 1) << 2;
    f32x4 f[IR][S];
#pragma unroll
    for (int ir = 0; ir < IR; ++ir) {
        const int ih = ih0 + ir;
        const bool row_ok = on && (unsigned)ih < (unsigned)d.h;
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int col = col0 + 4 * u;
            f[ir][u] = buf_f32x4(rx, (row_ok && col < d.w) ? (plane_off + (uint32_t)ih * d.w + col) * 4u : kOOB);
        }
    }
    // residual rows and the filter, in flight with the input rows
    const uint32_t out0 = (pl * (uint32_t)d.oh + (uint32_t)(b * RB)) * (uint32_t)d.ow + 4u * q;
    f32x4 rv[RB];
    if (VEC && res) {
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(res, (uint32_t)(((int64_t)d.n * d.c) * d.oh * d.ow * 4));
#pragma unroll
        for (int r = 0; r < RB; ++r)
            rv[r] = buf_f32x4(rr, (on && b * RB + r < d.oh) ? (out0 + (uint32_t)(r * d.ow)) * 4u : kOOB);
    } else {
#pragma unroll
        for (int r = 0; r < RB; ++r) rv[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float wk[K * K];
#pragma unroll
    for (int i = 0; i < K * K; ++i) wk[i] = w[c * K * K + i];
    float bv = bias ? bias[c] : 0.f;
    // Materialise the filter and bias here, while the input rows are in flight
    // (left alone, the compiler sinks their loads below the wait for the rows).
#pragma unroll
    for (int i = 0; i < K * K; ++i) asm volatile("" : "+s"(wk[i]));
    asm volatile("" : "+s"(bv));
    int act = d.act;
    asm volatile("" : "+s"(act));
    float acc[RB][4];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[r][j] = 0.f;
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
            v[j] = has_l ? t : 0.f;
        }
#pragma unroll
        for (int j = 0; j < HR; ++j) {
            const float t = __int_as_float(__builtin_amdgcn_ds_bpermute(addr_r, __float_as_int(f[ir][0][j])));
            v[HL + 4 * S + j] = has_r ? t : 0.f;
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int kh = ir - r * S;
            if (kh >= 0 && kh < K) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int kw = 0; kw < K; ++kw) acc[r][j] = fmaf(wk[kh * K + kw], v[j * S + kw], acc[r][j]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int oh = b * RB + r;
        if (!on || oh >= d.oh) break;
        const int ow0 = 4 * q;
        const uint32_t o = out0 + (uint32_t)(r * d.ow);
        if constexpr (VEC) {
            const f32x4 out = {apply_act(acc[r][0] + bv + rv[r][0], act), apply_act(acc[r][1] + bv + rv[r][1], act),
                               apply_act(acc[r][2] + bv + rv[r][2], act), apply_act(acc[r][3] + bv + rv[r][3], act)};
            // non-temporal: nothing in this launch reads the output again (measured on
            // YOLOv10n's batch-16 80 x 80 layers: 15.7 -> 13.5 us)
            __builtin_nontemporal_store(out, reinterpret_cast<f32x4 *>(y + o));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (ow0 + j < d.ow) {
                    float vv = acc[r][j] + bv;
                    if (res) vv += res[o + j];
                    y[o + j] = apply_act(vv, act);
                }
            }
        }
    }
}

template <int K, int S, int RB>
static int launch_dw_wave(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias,
                          const float *res, float *y, hipStream_t st) {
    const int owq = (d->ow + 3) / 4;
    const int bands = (d->oh + RB - 1) / RB;
    const int bpw = 64 / owq;
    const int wpp = (bands + bpw - 1) / bpw;
    const int64_t waves = (int64_t)d->n * d->c * wpp;
    constexpr int wpb = kDwWaveThreads / 64;
    const int64_t blocks = (waves + wpb - 1) / wpb;
    if (blocks * kDwWaveThreads > INT32_MAX) return SPINN_HIP_EUNSUPPORTED;
    const bool vec = d->ow % 4 == 0 && ((uintptr_t)y & 15u) == 0 && (!res || ((uintptr_t)res & 15u) == 0);
    if (vec)
        hipLaunchKernelGGL((dw_wave_kernel<K, S, RB, true>), dim3((unsigned)blocks), dim3(kDwWaveThreads), 0, st, x,
                           w, bias, res, y, *d, owq, bands, bpw, wpp, (int)waves);
    else
        hipLaunchKernelGGL((dw_wave_kernel<K, S, RB, false>), dim3((unsigned)blocks), dim3(kDwWaveThreads), 0, st, x,
                           w, bias, res, y, *d, owq, bands, bpw, wpp, (int)waves);
    return check_launch();
}

template <int K, int S, int RPT>
static int launch_dw_direct(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias,
                            const float *res, float *y, hipStream_t st) {
    const int owq = (d->ow + 3) / 4;
    const int row_groups = (d->oh + RPT - 1) / RPT;
    const int64_t total = (int64_t)d->n * d->c * row_groups * owq;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > INT32_MAX) return SPINN_HIP_EUNSUPPORTED;
    const bool vec = d->ow % 4 == 0 && ((uintptr_t)y & 15u) == 0 && (!res || ((uintptr_t)res & 15u) == 0);
    if (vec)
        hipLaunchKernelGGL((dw_direct_kernel<K, S, RPT, true>), dim3((unsigned)blocks), dim3(256), 0, st, x, w, bias,
                           res, y, *d, row_groups, owq, total);
    else
        hipLaunchKernelGGL((dw_direct_kernel<K, S, RPT, false>), dim3((unsigned)blocks), dim3(256), 0, st, x, w,
                           bias, res, y, *d, row_groups, owq, total);
    return check_launch();
}

static bool dw_direct_ok(const SpinnHipConvDesc *d) {
    static_assert(3 * 2 + 3 - 3 / 2 <= 8 && 3 + 7 - 7 / 2 <= 8, "three 16-byte loads cover the window");
    return d->w % 4 == 0 && d->pw == d->kw / 2 &&
           (int64_t)d->n * d->c * d->h * d->w * 4 <= (int64_t)kMaxOperandBytes;
}

// Stem convolutions with few input channels (RGB images): one thread per
// output pixel computes a chunk of 16 output channels, reading each input
// channel's KH x KW window into registers once and the chunk's weights from
// LDS (every lane reads the same word: a broadcast). The implicit GEMM would
// run these with K = C*KH*KW of 27..147 and mostly padded tiles.
constexpr int kStemOcb = 16;

template <int KH, int KW>
__global__ __launch_bounds__(256) void stem_conv_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                        const float *__restrict__ bias, const float *__restrict__ res,
                                                        float *__restrict__ y, SpinnHipConvDesc d) {
    __shared__ __attribute__((aligned(16))) float ws[kStemOcb * 4 * KH * KW];
    const int taps = d.c * KH * KW;
    const int oc0 = blockIdx.y * kStemOcb;
    const int ocn = min(kStemOcb, d.oc - oc0);
    for (int e = threadIdx.x; e < kStemOcb * taps; e += 256) {
        const int o = e / taps, t = e - o * taps;
        ws[t * kStemOcb + o] = o < ocn ? w[(int64_t)(oc0 + o) * taps + t] : 0.f;
    }
    __syncthreads();
    const int64_t ohw = (int64_t)d.oh * d.ow;
    const int64_t total = (int64_t)d.n * ohw;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t n = e / ohw;
        const int p = (int)(e - n * ohw);
        const int oh = p / d.ow, ow = p - oh * d.ow;
        const int ih0 = oh * d.sh - d.ph, iw0 = ow * d.sw - d.pw;
        float acc[kStemOcb];
#pragma unroll
        for (int o = 0; o < kStemOcb; ++o) acc[o] = 0.f;
        for (int c = 0; c < d.c; ++c) {
            const float *xc = x + (n * d.c + c) * (int64_t)d.h * d.w;
            float win[KH * KW];
#pragma unroll
            for (int kh = 0; kh < KH; ++kh)
#pragma unroll
                for (int kw = 0; kw < KW; ++kw) {
                    const int ih = ih0 + kh, iw = iw0 + kw;
                    win[kh * KW + kw] =
                        ((unsigned)ih < (unsigned)d.h && (unsigned)iw < (unsigned)d.w) ? xc[(int64_t)ih * d.w + iw] : 0.f;
                }
            const float *wc = ws + c * KH * KW * kStemOcb;
#pragma unroll
            for (int t = 0; t < KH * KW; ++t) {
#pragma unroll
                for (int o = 0; o < kStemOcb; o += 4) {
                    const float4 wv = *reinterpret_cast<const float4 *>(wc + t * kStemOcb + o);
                    acc[o + 0] = fmaf(wv.x, win[t], acc[o + 0]);
                    acc[o + 1] = fmaf(wv.y, win[t], acc[o + 1]);
                    acc[o + 2] = fmaf(wv.z, win[t], acc[o + 2]);
                    acc[o + 3] = fmaf(wv.w, win[t], acc[o + 3]);
                }
            }
        }
#pragma unroll
        for (int o = 0; o < kStemOcb; ++o) {
            if (o < ocn) {
                const int64_t idx = (n * d.oc + oc0 + o) * ohw + p;
                float v = acc[o];
                if (bias) v += bias[oc0 + o];
                if (res) v += res[idx];
                y[idx] = apply_act(v, d.act);
            }
        }
    }
}

bool stem_conv_eligible(const SpinnHipConvDesc *d) {
    return d->group == 1 && d->c <= 4 && ((d->kh == 3 && d->kw == 3) || (d->kh == 7 && d->kw == 7));
}

// Measured on MI355X: 2.6x the implicit GEMM for a 3x3 stem into 16 channels
// (YOLO, 640x640), while a 7x7 stem into 64 channels (ResNet) has enough K
// and M for the matrix cores to win.
bool stem_conv_pays(const SpinnHipConvDesc *d) { return stem_conv_eligible(d) && d->kh == 3 && d->oc <= 32; }

template <int K, int S>
static int launch_dw(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias, const float *res,
                     float *y, hipStream_t st) {
    const int tiles_h = (d->oh + kDwTH - 1) / kDwTH, tiles_w = (d->ow + kDwTW - 1) / kDwTW;
    const int64_t planes = (int64_t)d->n * d->c;
    const int64_t tiles = (int64_t)tiles_h * tiles_w;
    if (tiles >= 4) {
        // Measured on YOLOv10n batch 16: planes of >= 4 tiles gain from up to 4 planes per
        // workgroup with the next window prefetched (80x80: 22.1 -> 19.3 us, 80->40 stride 2:
        // 36.0 -> 29.4 us); one-tile planes lose, so they keep one plane per workgroup.
        const int64_t gy = std::min<int64_t>({planes, (int64_t)65535,
                                              std::max<int64_t>((planes + 3) / 4, (4096 + tiles - 1) / tiles)});
        hipLaunchKernelGGL((dw_tiled_kernel<K, S, true>), dim3((unsigned)tiles, (unsigned)gy), dim3(256), 0, st, x,
                           w, bias, res, y, *d, tiles_w, planes);
    } else {
        hipLaunchKernelGGL((dw_tiled_kernel<K, S, false>), dim3((unsigned)tiles, (unsigned)std::min<int64_t>(planes, 65535)),
                           dim3(256), 0, st, x, w, bias, res, y, *d, tiles_w, planes);
    }
    return check_launch();
}

int direct_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias, const float *res,
                float *y, hipStream_t st) {
    const int ohw = d->oh * d->ow;
    const bool depthwise = d->group == d->c && d->group == d->oc && d->kh == d->kw && d->sh == d->sw;
    if (depthwise && dw_direct_ok(d) && d->ow <= 256 && (d->kh == 3 || d->kh == 5 || d->kh == 7) &&
        (d->sh == 1 || (d->sh == 2 && d->kh == 3)) && d->ph == d->kh / 2) {
        // 3-row bands for rows of >= 64 pixels, 2-row bands below (measured on YOLOv10n's
        // batch-16 layers: 80 x 80 planes 10.6 -> 9.9 us with 3 rows, 20 x 20 and 40 x 40
        // planes slower by 0.4-0.8 us)
        if (d->kh == 3 && d->sh == 1 && d->ow >= 64) return launch_dw_wave<3, 1, 3>(d, x, w, bias, res, y, st);
        if (d->kh == 3 && d->sh == 1) return launch_dw_wave<3, 1, 2>(d, x, w, bias, res, y, st);
        if (d->kh == 3) return launch_dw_wave<3, 2, 1>(d, x, w, bias, res, y, st);
        if (d->kh == 5) return launch_dw_wave<5, 1, 2>(d, x, w, bias, res, y, st);
        return launch_dw_wave<7, 1, 2>(d, x, w, bias, res, y, st);
    }
    if (depthwise && dw_direct_ok(d) && (d->kh == 3 || d->kh == 5 || d->kh == 7) &&
        (d->sh == 1 || (d->sh == 2 && d->kh == 3))) {
        // Measured on YOLOv10n's 13 depthwise layers at batch 16: 114 us against 180 us for the
        // LDS-tiled kernel below and 162 us for LDS staging by asynchronous copies in two stages.
        if (d->kh == 3 && d->sh == 1) return launch_dw_direct<3, 1, 4>(d, x, w, bias, res, y, st);
        if (d->kh == 3) return launch_dw_direct<3, 2, 2>(d, x, w, bias, res, y, st);
        if (d->kh == 5) return launch_dw_direct<5, 1, 4>(d, x, w, bias, res, y, st);
        return launch_dw_direct<7, 1, 2>(d, x, w, bias, res, y, st);
    }
    if (depthwise && (int64_t)((d->oh + kDwTH - 1) / kDwTH) * ((d->ow + kDwTW - 1) / kDwTW) <= 65535) {
        if (d->kh == 3 && d->sh == 1) return launch_dw<3, 1>(d, x, w, bias, res, y, st);
        if (d->kh == 3 && d->sh == 2) return launch_dw<3, 2>(d, x, w, bias, res, y, st);
        if (d->kh == 5 && d->sh == 1) return launch_dw<5, 1>(d, x, w, bias, res, y, st);
        if (d->kh == 7 && d->sh == 1) return launch_dw<7, 1>(d, x, w, bias, res, y, st);
    }
    if (stem_conv_eligible(d)) {
        // Measured on YOLOv10n's 3 -> 16 stem at 640x640: 50.1 us against 53.5-55 us at batch 16
        // (5120 rows), 9.2 against 9.0 us at batch 1 (320 rows: too few workgroups to hide the
        // staging loads), so the MFMA kernel takes grids of at least 4 rows per CU.
        if (stem3_mfma_eligible(d) && (int64_t)d->n * d->oh >= 4 * (int64_t)device_cu_count())
            return stem3_mfma_conv(d, x, w, bias, res, y, st);
        const int64_t total = (int64_t)d->n * ohw;
        dim3 grid((unsigned)std::min<int64_t>((total + 255) / 256, 1 << 16), (unsigned)((d->oc + kStemOcb - 1) / kStemOcb));
        if (d->kh == 3)
            hipLaunchKernelGGL((stem_conv_kernel<3, 3>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
        else
            hipLaunchKernelGGL((stem_conv_kernel<7, 7>), grid, dim3(256), 0, st, x, w, bias, res, y, *d);
        return check_launch();
    }
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
