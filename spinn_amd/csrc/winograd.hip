// winograd.hip - Winograd F(2x2,3x3) convolution as 16 batched MFMA GEMMs.
//
// Same transform matrices as the reference (SPINN/run_time/ops/conv/winograd.c:23-67):
//   V = B^T d B (4x4 input patch), U = G g G^T (3x3 filter), Y = A^T M A (2x2 output),
//   M[a] = U[a] . V[a] for the 16 positions a of the 4x4 transform domain.
// The reference path is disabled (conv2d.c:155) and would apply ReLU only
// (winograd.c:199); here the full fused epilogue (bias, residual, ReLU/SiLU)
// runs in the output transform, and the batch is folded into the tile axis.
//
// Data layout in the workspace (all fp32):
//   V [16][C][T]   T = N * ceil(OH/2) * ceil(OW/2) output tiles, tile-contiguous
//   M [16][OC][T]
// U (packed weights) is [16][C][OC], OC contiguous, so the GEMM reads both
// operands k-major with 16-byte loads.
#include "spinn_hip_internal.h"

namespace spinn {

namespace {

struct WinoGeom {
    int N, C, H, W, OC, OH, OW, PH, PW, TH, TW;
    int64_t T;
};

WinoGeom wino_geom(const SpinnHipConvDesc *d) {
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
    g.TH = (d->oh + 1) / 2;
    g.TW = (d->ow + 1) / 2;
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

bool winograd_eligible(const SpinnHipConvDesc *d) {
    return d->kh == 3 && d->kw == 3 && d->sh == 1 && d->sw == 1 && d->group == 1 && d->oh >= 1 && d->ow >= 1;
}

int64_t winograd_packed_floats(const SpinnHipConvDesc *d) { return (int64_t)16 * d->c * d->oc; }

int winograd_pack(const SpinnHipConvDesc *d, const float *w, float *packed, hipStream_t st) {
    const int64_t total = (int64_t)d->oc * d->c;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 65535);
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
    gd.batch = 16;
    gd.stride_a = (int64_t)g.C * g.OC;
    gd.stride_b = (int64_t)g.C * g.T;
    gd.stride_y = (int64_t)g.OC * g.T;
    return gd;
}

size_t winograd_workspace_bytes(const SpinnHipConvDesc *d) {
    WinoGeom g = wino_geom(d);
    return ((size_t)16 * g.C * g.T + (size_t)16 * g.OC * g.T) * sizeof(float);
}

int winograd_conv(const SpinnHipConvDesc *d, const float *x, const float *packed, const float *bias,
                  const float *res, float *y, void *ws, size_t ws_bytes, hipStream_t st) {
    WinoGeom g = wino_geom(d);
    if (g.T > INT32_MAX) return SPINN_HIP_EUNSUPPORTED;
    if (!ws || ws_bytes < winograd_workspace_bytes(d)) return SPINN_HIP_EWORKSPACE;
    float *V = (float *)ws;
    float *Mt = V + (size_t)16 * g.C * g.T;
    {
        const int64_t total = (int64_t)g.C * g.T;
        const int blocks = (int)std::min<int64_t>((total + 255) / 256, 16384);
        hipLaunchKernelGGL(wino_input_kernel, dim3(blocks), dim3(256), 0, st, x, V, g);
        int rc = check_launch();
        if (rc) return rc;
    }
    SpinnHipGemmDesc gd = wino_gemm_desc(g);
    int rc = gemm_run(&gd, packed, V, nullptr, Mt, nullptr, 0, st);
    if (rc) return rc;
    const int64_t total = (int64_t)g.OC * g.T;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 16384);
    hipLaunchKernelGGL(wino_output_kernel, dim3(blocks), dim3(256), 0, st, Mt, bias, res, d->act, y, g);
    return check_launch();
}

} // namespace spinn
