// winograd.hip - Winograd convolution for 3x3 stride-1 layers as batched MFMA GEMMs.
//
// Two tile sizes (the caller's algorithm choice passes m = 2 or 4):
//   F(2x2,3x3): 4x4 input patches, 16 GEMMs - the reference's transform matrices
//               (SPINN/run_time/ops/conv/winograd.c:23-67);
//   F(4x4,3x3): 6x6 input patches, 36 GEMMs - the interpolation points 0, +-1, +-2
//               of Lavin & Gray, "Fast Algorithms for Convolutional Neural Networks"
//               (2015): 4x fewer multiplies than direct convolution instead of 2.25x,
//               and V / M are 2.25x the input / output instead of 4x.
//   V = B^T d B (input patch), U = G g G^T (3x3 filter), Y = A^T M A (output tile),
//   M[a] = U[a] . V[a] for every position a of the transform domain.
// The reference path is disabled (conv2d.c:155) and would apply ReLU only
// (winograd.c:199); here the full fused epilogue (bias, residual, ReLU/SiLU)
// runs in the output transform, and the batch is folded into the tile axis.
//
// Data layout in the workspace (all fp32), P = 16 or 36 transform positions:
//   V [P][C][T]   T = N * ceil(OH/m) * ceil(OW/m) output tiles, tile-contiguous
//   M [P][OC][T]
// U (packed weights) is [P][C][OC], OC contiguous, so the GEMM reads both
// operands k-major with 16-byte loads.
#include "spinn_hip_internal.h"
#include "winograd_tf.h"

namespace spinn {

namespace {

struct WinoGeom {
    int N, C, H, W, OC, OH, OW, PH, PW, TH, TW;
    int m, P; // output tile edge (2 or 4) and transform positions ((m + 2)^2)
    int64_t T;
};

WinoGeom wino_geom(const SpinnHipConvDesc *d, int m) {
    WinoGeom g;
    g.N = d->n;
    g.C = d->c;
    g.H = d->h;
    g.W = d->w;
    g.OC = d->oc;
    g.OH = d->oh;
    g.OW = d->ow;
    g.PH = d->ph;
    g.PW = d->pw;
    g.m = m;
    g.P = (g.m + 2) * (g.m + 2);
    g.TH = (d->oh + g.m - 1) / g.m;
    g.TW = (d->ow + g.m - 1) / g.m;
    g.T = (int64_t)g.N * g.TH * g.TW;
    return g;
}

} // namespace

// U[a][c][oc] = (G g G^T)[a] for g = w[oc][c] (3x3).
__global__ void wino_pack_kernel(const float *__restrict__ w, float *__restrict__ U, int OC, int C) {
    const int64_t total = (int64_t)OC * C;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(e / OC);
        const int oc = (int)(e - (int64_t)c * OC);
        const float *g = w + ((int64_t)oc * C + c) * 9;
        float t[4][3];
        for (int j = 0; j < 3; ++j) {
            t[0][j] = g[0 * 3 + j];
            t[1][j] = 0.5f * (g[0 * 3 + j] + g[1 * 3 + j] + g[2 * 3 + j]);
            t[2][j] = 0.5f * (g[0 * 3 + j] - g[1 * 3 + j] + g[2 * 3 + j]);
            t[3][j] = g[2 * 3 + j];
        }
        for (int i = 0; i < 4; ++i) {
            float u0 = t[i][0];
            float u1 = 0.5f * (t[i][0] + t[i][1] + t[i][2]);
            float u2 = 0.5f * (t[i][0] - t[i][1] + t[i][2]);
            float u3 = t[i][2];
            const int64_t base = (int64_t)c * OC + oc;
            U[(int64_t)(i * 4 + 0) * C * OC + base] = u0;
            U[(int64_t)(i * 4 + 1) * C * OC + base] = u1;
            U[(int64_t)(i * 4 + 2) * C * OC + base] = u2;
            U[(int64_t)(i * 4 + 3) * C * OC + base] = u3;
        }
    }
}

// One thread per (c, tile): V[a][c][t] = (B^T d B)[a].
__global__ __launch_bounds__(256) void wino_input_kernel(const float *__restrict__ x, float *__restrict__ V,
                                                         WinoGeom g) {
    const int64_t total = (int64_t)g.C * g.T;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(e / g.T);
        const int64_t t = e - (int64_t)c * g.T;
        const int per_img = g.TH * g.TW;
        const int n = (int)(t / per_img);
        const int r = (int)(t - (int64_t)n * per_img);
        const int ty = r / g.TW;
        const int tx = r - ty * g.TW;
        const int ih0 = 2 * ty - g.PH;
        const int iw0 = 2 * tx - g.PW;
        const float *xp = x + ((int64_t)n * g.C + c) * g.H * g.W;
        float d[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ih = ih0 + i, iw = iw0 + j;
                d[i][j] = ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                              ? xp[(int64_t)ih * g.W + iw]
                              : 0.f;
            }
        float tt[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            tt[0][j] = d[0][j] - d[2][j];
            tt[1][j] = d[1][j] + d[2][j];
            tt[2][j] = -d[1][j] + d[2][j];
            tt[3][j] = d[1][j] - d[3][j];
        }
        const int64_t plane = (int64_t)g.C * g.T;
        float *vp = V + (int64_t)c * g.T + t;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vp[(i * 4 + 0) * plane] = tt[i][0] - tt[i][2];
            vp[(i * 4 + 1) * plane] = tt[i][1] + tt[i][2];
            vp[(i * 4 + 2) * plane] = -tt[i][1] + tt[i][2];
            vp[(i * 4 + 3) * plane] = tt[i][1] - tt[i][3];
        }
    }
}

// One thread per (oc, tile): Y = A^T M A, then bias / residual / activation.
__global__ __launch_bounds__(256) void wino_output_kernel(const float *__restrict__ Mt,
                                                          const float *__restrict__ bias,
                                                          const float *__restrict__ res, int act,
                                                          float *__restrict__ y, WinoGeom g) {
    const int64_t total = (int64_t)g.OC * g.T;
    const int64_t plane = total;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int oc = (int)(e / g.T);
        const int64_t t = e - (int64_t)oc * g.T;
        float m[4][4];
#pragma unroll
        for (int a = 0; a < 16; ++a) m[a / 4][a % 4] = Mt[a * plane + e];
        float tt[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            tt[0][j] = m[0][j] + m[1][j] + m[2][j];
            tt[1][j] = m[1][j] - m[2][j] - m[3][j];
        }
        float o[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            o[i][0] = tt[i][0] + tt[i][1] + tt[i][2];
            o[i][1] = tt[i][1] - tt[i][2] - tt[i][3];
        }
        const int per_img = g.TH * g.TW;
        const int n = (int)(t / per_img);
        const int r = (int)(t - (int64_t)n * per_img);
        const int ty = r / g.TW;
        const int tx = r - ty * g.TW;
        const float b = bias ? bias[oc] : 0.f;
        const int64_t ybase = ((int64_t)n * g.OC + oc) * g.OH * g.OW;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int oh = 2 * ty + i, ow = 2 * tx + j;
                if (oh < g.OH && ow < g.OW) {
                    const int64_t idx = ybase + (int64_t)oh * g.OW + ow;
                    float v = o[i][j] + b;
                    if (res) v += res[idx];
                    y[idx] = apply_act(v, act);
                }
            }
    }
}

// F(4,3): U[a][c][oc] = (G g G^T)[a], a = 6 * row + col.
__global__ void wino4_pack_kernel(const float *__restrict__ w, float *__restrict__ U, int OC, int C) {
    const int64_t total = (int64_t)OC * C;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(e / OC);
        const int oc = (int)(e - (int64_t)c * OC);
        const float *g = w + ((int64_t)oc * C + c) * 9;
        float t[6][3]; // G g: 6 rows of 3
        for (int j = 0; j < 3; ++j) {
            const float col[3] = {g[j], g[3 + j], g[6 + j]};
            float o[6];
            g6(col, o);
            for (int i = 0; i < 6; ++i) t[i][j] = o[i];
        }
        const int64_t plane = (int64_t)C * OC, base = (int64_t)c * OC + oc;
        for (int i = 0; i < 6; ++i) {
            float o[6];
            g6(t[i], o);
            for (int j = 0; j < 6; ++j) U[(int64_t)(i * 6 + j) * plane + base] = o[j];
        }
    }
}

// F(4,3) transforms: a workgroup takes 64 consecutive tiles of one channel with 6 threads
// per tile (384 threads, one wave per patch column / row). Phase 1 transforms the 6
// columns of every patch, phase 2 - after an exchange through LDS - its rows, so each
// thread issues 6 loads and 6 stores and every wave's accesses cover 64 consecutive tiles.
constexpr int kW4Tiles = 64;
constexpr int kW4Threads = 6 * kW4Tiles;

// V[a][c][t] = (B^T d B)[a] over the 6x6 input patch of tile t. Grid: (ceil(T / 64), C).
__global__ __launch_bounds__(kW4Threads) void wino4_input_kernel(const float *__restrict__ x,
                                                                 float *__restrict__ V, WinoGeom g) {
    // [tile][row i][column j]; a tile's 42 words padded to an odd stride, so the 64
    // lanes of a wave (64 tiles) fall in 64 different banks
    constexpr int kTS = 43;
    __shared__ float tt[kW4Tiles * kTS];
    const int lane_t = threadIdx.x % kW4Tiles;
    const int q = threadIdx.x / kW4Tiles; // phase 1: patch column j; phase 2: transform row i
    const int c = blockIdx.y;
    const int64_t t = (int64_t)blockIdx.x * kW4Tiles + lane_t;
    const bool live = t < g.T;
    if (live) {
        const int per_img = g.TH * g.TW;
        const int n = (int)(t / per_img);
        const int r = (int)(t - (int64_t)n * per_img);
        const int ty = r / g.TW;
        const int tx = r - ty * g.TW;
        const int ih0 = 4 * ty - g.PH;
        const int iw = 4 * tx - g.PW + q;
        const float *xp = x + ((int64_t)n * g.C + c) * g.H * g.W;
        const bool col_in = (unsigned)iw < (unsigned)g.W;
        float col[6];
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            const int ih = ih0 + i;
            col[i] = (col_in && (unsigned)ih < (unsigned)g.H) ? xp[(int64_t)ih * g.W + iw] : 0.f;
        }
        float o[6];
        bt6(col, o);
#pragma unroll
        for (int i = 0; i < 6; ++i) tt[lane_t * kTS + i * 7 + q] = o[i];
    }
    __syncthreads();
    if (live) {
        float row[6];
#pragma unroll
        for (int j = 0; j < 6; ++j) row[j] = tt[lane_t * kTS + q * 7 + j];
        float o[6];
        bt6(row, o);
        const int64_t plane = (int64_t)g.C * g.T;
        float *vp = V + (int64_t)(q * 6) * plane + (int64_t)c * g.T + t;
#pragma unroll
        for (int j = 0; j < 6; ++j) vp[(int64_t)j * plane] = o[j];
    }
}

// Y = A^T M A (4x4 output tile), then bias / residual / activation. Grid: (ceil(T / 64), OC).
// Phase 1: 6 threads per tile transform the columns of M (6 -> 4 values each); phase 2: 4 of
// them transform the rows and write one output row of 4 pixels each.
__global__ __launch_bounds__(kW4Threads) void wino4_output_kernel(const float *__restrict__ Mt,
                                                                  const float *__restrict__ bias,
                                                                  const float *__restrict__ res, int act,
                                                                  float *__restrict__ y, WinoGeom g) {
    // [tile][row i][column j]; a tile's 28 words padded to an odd stride (conflict-free)
    constexpr int kTS = 29;
    __shared__ float tt[kW4Tiles * kTS];
    const int lane_t = threadIdx.x % kW4Tiles;
    const int q = threadIdx.x / kW4Tiles;
    const int oc = blockIdx.y;
    const int64_t t = (int64_t)blockIdx.x * kW4Tiles + lane_t;
    const bool live = t < g.T;
    const int64_t plane = (int64_t)g.OC * g.T;
    if (live) {
        const float *mp = Mt + (int64_t)oc * g.T + t;
        float col[6];
#pragma unroll
        for (int i = 0; i < 6; ++i) col[i] = mp[(int64_t)(i * 6 + q) * plane];
        float o[4];
        at6(col, o);
#pragma unroll
        for (int i = 0; i < 4; ++i) tt[lane_t * kTS + i * 7 + q] = o[i];
    }
    __syncthreads();
    if (live && q < 4) {
        float row[6];
#pragma unroll
        for (int j = 0; j < 6; ++j) row[j] = tt[lane_t * kTS + q * 7 + j];
        float o[4];
        at6(row, o);
        const int per_img = g.TH * g.TW;
        const int n = (int)(t / per_img);
        const int r = (int)(t - (int64_t)n * per_img);
        const int ty = r / g.TW;
        const int tx = r - ty * g.TW;
        const int oh = 4 * ty + q;
        if (oh < g.OH) {
            const float b = bias ? bias[oc] : 0.f;
            const int64_t base = (((int64_t)n * g.OC + oc) * g.OH + oh) * g.OW;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ow = 4 * tx + j;
                if (ow < g.OW) {
                    float v = o[j] + b;
                    if (res) v += res[base + ow];
                    y[base + ow] = apply_act(v, act);
                }
            }
        }
    }
}

bool winograd_eligible(const SpinnHipConvDesc *d) {
    return d->kh == 3 && d->kw == 3 && d->sh == 1 && d->sw == 1 && d->group == 1 && d->oh >= 1 && d->ow >= 1;
}

int64_t winograd_packed_floats(const SpinnHipConvDesc *d, int m) {
    const int a = m + 2;
    return (int64_t)a * a * d->c * d->oc;
}

int winograd_pack(const SpinnHipConvDesc *d, int m, const float *w, float *packed, hipStream_t st) {
    const int64_t total = (int64_t)d->oc * d->c;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 65535);
    if (m == 4)
        hipLaunchKernelGGL(wino4_pack_kernel, dim3(blocks), dim3(256), 0, st, w, packed, d->oc, d->c);
    else
        hipLaunchKernelGGL(wino_pack_kernel, dim3(blocks), dim3(256), 0, st, w, packed, d->oc, d->c);
    return check_launch();
}

static SpinnHipGemmDesc wino_gemm_desc(const WinoGeom &g) {
    SpinnHipGemmDesc gd{};
    gd.m = g.OC;
    gd.n = (int32_t)g.T;
    gd.k = g.C;
    gd.trans_a = 1; // U[a] stored [C][OC]
    gd.trans_b = 0; // V[a] stored [C][T]
    gd.c_mode = 0;
    gd.alpha = 1.f;
    gd.beta = 0.f;
    gd.batch = g.P;
    gd.stride_a = (int64_t)g.C * g.OC;
    gd.stride_b = (int64_t)g.C * g.T;
    gd.stride_y = (int64_t)g.OC * g.T;
    return gd;
}

size_t winograd_workspace_bytes(const SpinnHipConvDesc *d, int m) {
    if (m == 4 && wino4_fused_selected(d)) return 0; // V and M stay on chip
    WinoGeom g = wino_geom(d, m);
    return ((size_t)g.P * g.C * g.T + (size_t)g.P * g.OC * g.T) * sizeof(float);
}

int winograd_conv(const SpinnHipConvDesc *d, int m, const float *x, const float *packed, const float *bias,
                  const float *res, float *y, void *ws, size_t ws_bytes, hipStream_t st) {
    if (m == 4 && wino4_fused_selected(d)) return wino4_fused_conv(d, x, packed, bias, res, y, st);
    WinoGeom g = wino_geom(d, m);
    if (g.T > INT32_MAX) return SPINN_HIP_EUNSUPPORTED;
    if (m == 4 && (g.C > 65535 || g.OC > 65535)) return SPINN_HIP_EUNSUPPORTED; // channels on grid y
    if (!ws || ws_bytes < winograd_workspace_bytes(d, m)) return SPINN_HIP_EWORKSPACE;
    float *V = (float *)ws;
    float *Mt = V + (size_t)g.P * g.C * g.T;
    {
        const int64_t total = (int64_t)g.C * g.T;
        const int blocks = (int)std::min<int64_t>((total + 255) / 256, 16384);
        if (g.m == 4)
            hipLaunchKernelGGL(wino4_input_kernel, dim3((unsigned)((g.T + kW4Tiles - 1) / kW4Tiles), g.C),
                               dim3(kW4Threads), 0, st, x, V, g);
        else
            hipLaunchKernelGGL(wino_input_kernel, dim3(blocks), dim3(256), 0, st, x, V, g);
        int rc = check_launch();
        if (rc) return rc;
    }
    SpinnHipGemmDesc gd = wino_gemm_desc(g);
    int rc = gemm_run(&gd, packed, V, nullptr, Mt, nullptr, 0, st);
    if (rc) return rc;
    const int64_t total = (int64_t)g.OC * g.T;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 16384);
    if (g.m == 4)
        hipLaunchKernelGGL(wino4_output_kernel, dim3((unsigned)((g.T + kW4Tiles - 1) / kW4Tiles), g.OC),
                           dim3(kW4Threads), 0, st, Mt, bias, res, d->act, y, g);
    else
        hipLaunchKernelGGL(wino_output_kernel, dim3(blocks), dim3(256), 0, st, Mt, bias, res, d->act, y, g);
    return check_launch();
}

} // namespace spinn
