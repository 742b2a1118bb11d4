// mfma_core.h - fp32 MFMA tile engine for gfx950 (CDNA4, wave64).
//
// One workgroup = 256 threads = 4 waves arranged 2x2 over a BM x BN output
// tile. Each wave owns a (BM/2) x (BN/2) sub-tile made of 32x32 blocks computed
// with v_mfma_f32_32x32x2f32 (4096 flop per instruction, 64 cycles, the full
// fp32 matrix rate of a SIMD). The K loop stages BK-deep slices of both
// operands through LDS, double buffered: the next slice is fetched into
// registers while the current one feeds the matrix cores, then written to the
// other LDS buffer, one barrier per slice.
//
// LDS layout of both operands is k-major, [BK][BT + PAD] with T (the M or N
// index) contiguous, so the operand fetch of an MFMA (lane l reads element
// (k = 2s + l/32, t = t0 + l%32)) is 32 consecutive words per half-wave; PAD
// puts the two half-waves 32 banks apart.
//
// MFMA 32x32x2 f32 register layout (CDNA3/CDNA4 ISA, matrix instruction
// tables): A operand lane l = A[l%32][l/32], B operand lane l = B[l/32][l%32],
// accumulator element r of lane l = D[8*(r/4) + 4*(l/32) + r%4][l%32].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spinn {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

template <int BT>
struct LdsPad {
    // Row stride of a k-major LDS tile: keep it a multiple of 4 floats (b128
    // stores) and 32 words off a multiple of 64 so the two half-waves of an
    // operand fetch land in disjoint banks.
    static constexpr int value = ((BT % 64) == 0) ? 32 : (((BT + 32) % 64 == 0) ? 0 : 32 - (BT % 32));
    static constexpr int stride = BT + value;
};

template <int BM, int BN>
struct WaveTiling {
    static constexpr int WM = BM / 2;  // rows per wave
    static constexpr int WN = BN / 2;  // cols per wave
    static constexpr int TM = WM / 32; // 32x32 blocks per wave along M
    static constexpr int TN = WN / 32;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32x32");
};

// acc += A_lds[k-slice] x B_lds[k-slice] for one BK slice.
template <int BM, int BN, int BK>
__device__ __forceinline__ void mma_slice(const float *__restrict__ As, const float *__restrict__ Bs,
                                          f32x16 (&acc)[WaveTiling<BM, BN>::TM][WaveTiling<BM, BN>::TN],
                                          int wm0, int wn0, int lane) {
    constexpr int SA = LdsPad<BM>::stride;
    constexpr int SB = LdsPad<BN>::stride;
    constexpr int TM = WaveTiling<BM, BN>::TM;
    constexpr int TN = WaveTiling<BM, BN>::TN;
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const float *ap = As + h * SA + wm0 + l32;
    const float *bp = Bs + h * SB + wn0 + l32;
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
        float a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = ap[(2 * s) * SA + i * 32];
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = bp[(2 * s) * SB + j * 32];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// ---------------------------------------------------------------------------
// Tile loaders. Each stages a BK x BT slice of one operand: fetch() issues the
// global loads into registers for slice [k0, k0+BK), commit() writes them to
// a k-major LDS buffer. Elements outside [0,T) x [k_begin,k_end) are zero.
// ---------------------------------------------------------------------------

// Source laid out [K][ld] with the tile index contiguous (packed conv weights
// W^T, a transposed Gemm A, a plain Gemm B). VEC: float4 along T, which needs
// ld % 4 == 0, a 16-byte aligned base and T padded to a multiple of 4.
template <int BT, int BK, bool VEC>
struct KMajorLoader {
    static constexpr int S = LdsPad<BT>::stride;
    static constexpr int NV = VEC ? (BK * BT / 4) / kThreads : (BK * BT) / kThreads;
    static_assert(NV >= 1, "tile too small for 256 threads");
    const float *src; // already offset to (batch/group) and tile start t0
    int64_t ld;
    int t_valid;      // T - t0 (elements of the tile that exist)
    int k_end;
    f32x4 rv[VEC ? NV : 1];
    float rs[VEC ? 1 : NV];

    __device__ __forceinline__ void fetch(int k0, int tid) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                int c = tid + i * kThreads;
                int k = c / (BT / 4);
                int t = (c % (BT / 4)) * 4;
                int kk = k0 + k;
                if (kk < k_end && t < t_valid)
                    rv[i] = *reinterpret_cast<const f32x4 *>(src + (int64_t)kk * ld + t);
                else
                    rv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                int e = tid + i * kThreads;
                int k = e / BT;
                int t = e % BT;
                int kk = k0 + k;
                rs[i] = (kk < k_end && t < t_valid) ? src[(int64_t)kk * ld + t] : 0.f;
            }
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                int c = tid + i * kThreads;
                int k = c / (BT / 4);
                int t = (c % (BT / 4)) * 4;
                *reinterpret_cast<f32x4 *>(lds + k * S + t) = rv[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                int e = tid + i * kThreads;
                lds[(e / BT) * S + (e % BT)] = rs[i];
            }
        }
    }
};

// Source laid out [T][ld] with K contiguous (a plain Gemm A, a transposed
// Gemm B). Each thread reads 4 consecutive k of one row (float4 when VEC:
// ld % 4 == 0 and aligned base) and scatters them to 4 LDS rows; consecutive
// lanes take consecutive rows so the LDS writes are conflict-free.
template <int BT, int BK, bool VEC>
struct RowKLoader {
    static constexpr int S = LdsPad<BT>::stride;
    static constexpr int NQ = (BK / 4) * BT / kThreads; // float4 groups per thread
    static_assert(NQ >= 1 && BK % 4 == 0, "tile too small");
    const float *src;
    int64_t ld;
    int t_valid;
    int k_end;
    f32x4 r[NQ];

    __device__ __forceinline__ void fetch(int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            int c = tid + i * kThreads;
            int t = c % BT;
            int kq = (c / BT) * 4;
            int kk = k0 + kq;
            const float *p = src + (int64_t)t * ld + kk;
            if (t < t_valid && kk + 3 < k_end) {
                if constexpr (VEC) {
                    r[i] = *reinterpret_cast<const f32x4 *>(p);
                } else {
                    r[i] = f32x4{p[0], p[1], p[2], p[3]};
                }
            } else {
                f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (t < t_valid) {
                    if (kk + 0 < k_end) v[0] = p[0];
                    if (kk + 1 < k_end) v[1] = p[1];
                    if (kk + 2 < k_end) v[2] = p[2];
                }
                r[i] = v;
            }
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            int c = tid + i * kThreads;
            int t = c % BT;
            int kq = (c / BT) * 4;
            lds[(kq + 0) * S + t] = r[i][0];
            lds[(kq + 1) * S + t] = r[i][1];
            lds[(kq + 2) * S + t] = r[i][2];
            lds[(kq + 3) * S + t] = r[i][3];
        }
    }
};

// Geometry of the implicit-GEMM B operand: column j of the GEMM is output
// pixel (img, oh, ow) = (j / OHW, (j % OHW) / OW, j % OW); row k is a tap
// (c, kh, kw) of the convolution window.
struct ConvGeom {
    const float *x; // input of group 0, image 0
    int C, H, W;    // full input tensor dims
    int Cg;         // input channels per group
    int OH, OW;
    int KH, KW, SH, SW, PH, PW;
    int ntot;       // N * OH * OW
};

// im2col gather, K in (c, kh, kw) order - the row order of the reference's
// im2col (SPINN/run_time/ops/conv/conv2d.c:58-76). Any shape; per element it
// decomposes k with compile-time KH, KW (KHW = KH*KW, 0 = runtime).
template <int BN, int BK, int KHC, int KWC>
struct Im2colLoader {
    static constexpr int S = LdsPad<BN>::stride;
    static constexpr int NV = BK * BN / kThreads;
    static constexpr int KSTEP = kThreads / BN;
    static_assert(kThreads % BN == 0, "BN must divide 256");
    ConvGeom g;
    const float *base; // this thread's image (and group) base, or null if the column is out of range
    int ih0, iw0;
    int k_end;
    float r[NV];

    __device__ __forceinline__ void init(const ConvGeom &geom, int n0, int group, int tid, int kend) {
        g = geom;
        k_end = kend;
        int j = n0 + (tid % BN);
        int ohw = g.OH * g.OW;
        if (j < g.ntot) {
            int img = j / ohw;
            int p = j - img * ohw;
            int oh = p / g.OW;
            int ow = p - oh * g.OW;
            ih0 = oh * g.SH - g.PH;
            iw0 = ow * g.SW - g.PW;
            base = g.x + ((int64_t)img * g.C + (int64_t)group * g.Cg) * g.H * g.W;
        } else {
            base = nullptr;
            ih0 = iw0 = 0;
        }
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
        const int KH = KHC > 0 ? KHC : g.KH;
        const int KW = KWC > 0 ? KWC : g.KW;
        const int KHW = KH * KW;
        const int kt = tid / BN;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            int k = k0 + kt + i * KSTEP;
            float v = 0.f;
            if (base && k < k_end) {
                int c = k / KHW;
                int rr = k - c * KHW;
                int kh = rr / KW;
                int kw = rr - kh * KW;
                int ih = ih0 + kh;
                int iw = iw0 + kw;
                if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                    v = base[((int64_t)c * g.H + ih) * g.W + iw];
            }
            r[i] = v;
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
        const int kt = tid / BN;
        const int n = tid % BN;
#pragma unroll
        for (int i = 0; i < NV; ++i) lds[(kt + i * KSTEP) * S + n] = r[i];
    }
};

// im2col gather, K in (kh, kw, c) order; needs Cg % BK == 0 so one BK slice is
// a single tap (kh, kw) over BK consecutive channels: one bounds check per
// thread per slice, then BK/KSTEP strided loads.
template <int BN, int BK>
struct Im2colTapLoader {
    static constexpr int S = LdsPad<BN>::stride;
    static constexpr int NV = BK * BN / kThreads;
    static constexpr int KSTEP = kThreads / BN;
    ConvGeom g;
    const float *base;
    int ih0, iw0;
    int64_t hw;
    float r[NV];

    __device__ __forceinline__ void init(const ConvGeom &geom, int n0, int group, int tid, int /*kend*/) {
        g = geom;
        hw = (int64_t)g.H * g.W;
        int j = n0 + (tid % BN);
        int ohw = g.OH * g.OW;
        if (j < g.ntot) {
            int img = j / ohw;
            int p = j - img * ohw;
            int oh = p / g.OW;
            int ow = p - oh * g.OW;
            ih0 = oh * g.SH - g.PH;
            iw0 = ow * g.SW - g.PW;
            base = g.x + ((int64_t)img * g.C + (int64_t)group * g.Cg) * hw;
        } else {
            base = nullptr;
            ih0 = iw0 = 0;
        }
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
        const int tap = k0 / g.Cg;
        const int c0 = k0 - tap * g.Cg;
        const int kh = tap / g.KW;
        const int kw = tap - kh * g.KW;
        const int ih = ih0 + kh;
        const int iw = iw0 + kw;
        const bool ok = base && (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
        const float *p = ok ? base + (int64_t)(c0 + tid / BN) * hw + (int64_t)ih * g.W + iw : nullptr;
#pragma unroll
        for (int i = 0; i < NV; ++i) r[i] = ok ? p[(int64_t)i * KSTEP * hw] : 0.f;
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
        const int kt = tid / BN;
        const int n = tid % BN;
#pragma unroll
        for (int i = 0; i < NV; ++i) lds[(kt + i * KSTEP) * S + n] = r[i];
    }
};

} // namespace spinn
