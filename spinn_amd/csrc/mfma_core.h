// mfma_core.h - fp32 MFMA tile engine for gfx950 (CDNA4, wave64).
//
// One workgroup = 256 threads = 4 waves arranged 2x2 (1x4 for 32-row tiles)
// over a BM x BN output tile. Each wave owns a sub-tile made of 32x32 blocks computed
// with v_mfma_f32_32x32x2f32 (4096 flop per instruction, 64 cycles, the full
// fp32 matrix rate of a SIMD). The K loop stages BK-deep slices of both
// operands through two LDS buffers and NS register stages (gemm_mainloop).
//
// LDS layout of both operands is k-major, [BK][BT (+ PAD)] with T (the M or N
// index) contiguous, so the operand fetch of an MFMA (lane l reads element
// (k = 2s + l/32, t = t0 + l%32)) is 32 consecutive words per half-wave; a
// swizzle of odd rows (or PAD) puts the two half-waves 32 banks apart.
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
    // Row stride and column placement of a k-major LDS tile. The two
    // half-waves of an operand fetch read rows k and k+1 and must land in
    // disjoint halves of the 64 banks. Tiles 64 or 128 wide are unpadded and
    // store column t of odd rows at t ^ 32 (the swizzle keeps every aligned
    // float4 contiguous); other widths pad the row to 32 words off a multiple
    // of 64 (a 32-wide tile needs no pad).
    static constexpr bool swz = (BT % 64) == 0;
    static constexpr int value = swz ? 0 : (((BT + 32) % 64 == 0) ? 0 : 32 - (BT % 32));
    static constexpr int stride = BT + value;
    __device__ static __forceinline__ int col(int k, int t) { return swz ? (t ^ ((k & 1) << 5)) : t; }
};

// The 4 waves of a workgroup sit 2x2 over the tile, or 1x4 when the tile is
// only 32 rows tall (small-OC convs); wave w starts at (origin_m, origin_n).
template <int BM, int BN>
struct WaveTiling {
    static constexpr int WAVES_M = BM >= 64 ? 2 : 1;
    static constexpr int WAVES_N = 4 / WAVES_M;
    static constexpr int WM = BM / WAVES_M; // rows per wave
    static constexpr int WN = BN / WAVES_N; // cols per wave
    static constexpr int TM = WM / 32;      // 32x32 blocks per wave along M
    static constexpr int TN = WN / 32;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32x32");
    __device__ static int origin_m(int wave) { return (wave / WAVES_N) * WM; }
    __device__ static int origin_n(int wave) { return (wave % WAVES_N) * WN; }
};

// Accumulator start value of the plain GEMM: zero.
struct ZeroAcc {
    template <class Acc>
    __device__ __forceinline__ void operator()(Acc &acc) const {
        constexpr int N = sizeof(Acc) / sizeof(f32x16);
        f32x16 *p = reinterpret_cast<f32x16 *>(&acc);
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) p[i][r] = 0.f;
    }
};

// ---------------------------------------------------------------------------
// Tile loaders. Each stages a BK x BT slice of one operand: fetch() issues the
// global loads into registers for slice [k0, k0+BK), commit() writes them to
// a k-major LDS buffer.
//
// All loads are raw buffer loads through a resource descriptor whose size is
// the operand's extent: an offset at or past it returns 0 in hardware. Every
// element that must read as zero (conv padding, tile edges, the K tail) gets
// the offset kOOB instead of a branch, so the loads are unconditional and the
// compiler can wait on exactly the pipeline stage it needs.
// ---------------------------------------------------------------------------
constexpr uint32_t kOOB = 0x80000000u;         // any offset >= the operand's byte size
constexpr uint32_t kMaxOperandBytes = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, uint32_t bytes) {
    // dword3 0x00020000: 32-bit data format, the gfx9-family raw-buffer setting
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buf_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ f32x4 buf_f32x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Source laid out [K][ld] with the tile index contiguous (packed conv weights
// W^T, a transposed Gemm A, a plain Gemm B); `bytes` covers rows [0, K).
// VEC: float4 along T, which needs ld % 4 == 0, a 16-byte aligned base and a
// tile width T that is a multiple of 4 (or zero-padded to one).
// A tile of fewer elements than threads (VEC: fewer float4s) has the spare
// threads repeat the first ones: they load and store the same values to the
// same LDS words, which keeps every load unconditional.
template <int BT, int BK, bool VEC>
struct KMajorLoader {
    static constexpr bool kIsKMajor = true;
    static constexpr int S = LdsPad<BT>::stride;
    static constexpr int ITEMS = VEC ? BK * BT / 4 : BK * BT; // float4s (VEC) or floats per slice
    static constexpr int NV = ITEMS >= kThreads ? ITEMS / kThreads : 1;
    static_assert(ITEMS % kThreads == 0 || kThreads % ITEMS == 0, "tile does not map onto 256 threads");
    __device__ static int item(int tid, int i) { return ITEMS >= kThreads ? tid + i * kThreads : tid % ITEMS; }
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t ld;
    uint32_t t0;  // first tile index (m0 or n0)
    int t_valid;  // elements of the tile that exist: T - t0
    f32x4 rv[VEC ? NV : 1];
    float rs[VEC ? 1 : NV];

    __device__ __forceinline__ void init(const float *base, uint32_t bytes, uint32_t ld_, int t0_, int t_total) {
        rsrc = make_rsrc(base, bytes);
        ld = ld_;
        t0 = (uint32_t)t0_;
        t_valid = t_total - t0_;
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = item(tid, i);
                const int k = c / (BT / 4);
                const int t = (c % (BT / 4)) * 4;
                const uint32_t off = t < t_valid ? ((uint32_t)(k0 + k) * ld + t0 + t) * 4u : kOOB;
                rv[i] = buf_f32x4(rsrc, off);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int e = item(tid, i);
                const int k = e / BT;
                const int t = e % BT;
                const uint32_t off = t < t_valid ? ((uint32_t)(k0 + k) * ld + t0 + t) * 4u : kOOB;
                rs[i] = buf_f32(rsrc, off);
            }
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = item(tid, i);
                const int k = c / (BT / 4);
                *reinterpret_cast<f32x4 *>(lds + k * S + LdsPad<BT>::col(k, (c % (BT / 4)) * 4)) = rv[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int e = item(tid, i);
                lds[(e / BT) * S + LdsPad<BT>::col(e / BT, e % BT)] = rs[i];
            }
        }
    }
};

// Source laid out [T][ld] with K contiguous (a plain Gemm A, a transposed
// Gemm B); `bytes` covers rows [0, T). Each thread reads 4 consecutive k of
// one row (float4 when VEC: ld % 4 == 0 and an aligned base) and scatters
// them to 4 LDS rows; consecutive lanes take consecutive rows so the LDS
// writes are conflict-free. k >= k_end reads 0.
template <int BT, int BK, bool VEC>
struct RowKLoader {
    static constexpr bool kIsKMajor = false;
    static constexpr int S = LdsPad<BT>::stride;
    static constexpr int ITEMS = (BK / 4) * BT; // float4 row pieces per slice
    static constexpr int NQ = ITEMS >= kThreads ? ITEMS / kThreads : 1;
    static_assert(BK % 4 == 0 && (ITEMS % kThreads == 0 || kThreads % ITEMS == 0), "tile does not map onto 256 threads");
    // spare threads of a small tile repeat the first ones (same loads, same LDS words)
    __device__ static int item(int tid, int i) { return ITEMS >= kThreads ? tid + i * kThreads : tid % ITEMS; }
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t ld;
    uint32_t t0;
    int t_valid;
    int k_end;
    f32x4 r[NQ];

    __device__ __forceinline__ void init(const float *base, uint32_t bytes, uint32_t ld_, int t0_, int t_total,
                                         int kend) {
        rsrc = make_rsrc(base, bytes);
        ld = ld_;
        t0 = (uint32_t)t0_;
        t_valid = t_total - t0_;
        k_end = kend;
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int c = item(tid, i);
            const int t = c % BT;
            const int kk = k0 + (c / BT) * 4;
            const uint32_t row = (t0 + t) * ld;
            if constexpr (VEC) {
                // ld % 4 == 0 makes k_end - kk a multiple of 4 too, except at a
                // split-K chunk end, which is a multiple of 16
                r[i] = buf_f32x4(rsrc, (t < t_valid && kk < k_end) ? (row + kk) * 4u : kOOB);
            } else {
                f32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = buf_f32(rsrc, (t < t_valid && kk + e < k_end) ? (row + kk + e) * 4u : kOOB);
                r[i] = v;
            }
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int c = item(tid, i);
            const int t = c % BT;
            const int kq = (c / BT) * 4;
            lds[(kq + 0) * S + LdsPad<BT>::col(kq + 0, t)] = r[i][0];
            lds[(kq + 1) * S + LdsPad<BT>::col(kq + 1, t)] = r[i][1];
            lds[(kq + 2) * S + LdsPad<BT>::col(kq + 2, t)] = r[i][2];
            lds[(kq + 3) * S + LdsPad<BT>::col(kq + 3, t)] = r[i][3];
        }
    }
};

// Geometry of the implicit-GEMM B operand: column j of the GEMM is output
// pixel (img, oh, ow) = (j / OHW, (j % OHW) / OW, j % OW); row k is a tap
// (c, kh, kw) of the convolution window.
struct ConvGeom {
    const float *x; // input tensor base
    uint32_t x_bytes;
    int C, H, W;    // full input tensor dims
    int Cg;         // input channels per group
    int OH, OW;
    int KH, KW, SH, SW, PH, PW;
    int ntot;       // N * OH * OW
};

// Per-thread output pixel of a gather loader: element offset of its image
// (and group) plane and the window origin; `valid` false past the last pixel.
struct PixelOrigin {
    uint32_t base;
    int ih0, iw0;
    bool valid;
    __device__ __forceinline__ void init(const ConvGeom &g, int j, int group) {
        const int ohw = g.OH * g.OW;
        valid = j < g.ntot;
        const int jj = valid ? j : 0;
        const int img = jj / ohw;
        const int p = jj - img * ohw;
        const int oh = p / g.OW;
        const int ow = p - oh * g.OW;
        ih0 = oh * g.SH - g.PH;
        iw0 = ow * g.SW - g.PW;
        base = ((uint32_t)img * g.C + (uint32_t)group * g.Cg) * (uint32_t)(g.H * g.W);
    }
};

// im2col gather, K in (c, kh, kw) order - the row order of the reference's
// im2col (SPINN/run_time/ops/conv/conv2d.c:58-76). Any shape; per element it
// decomposes k with compile-time KH, KW when given (0 = runtime).
template <int BN, int BK, int KHC, int KWC>
struct Im2colLoader {
    static constexpr int S = LdsPad<BN>::stride;
    static constexpr int NV = BK * BN / kThreads;
    static constexpr int KSTEP = kThreads / BN;
    static_assert(kThreads % BN == 0, "BN must divide 256");
    __amdgpu_buffer_rsrc_t rsrc;
    ConvGeom g;
    PixelOrigin px;
    int k_end;
    float r[NV];

    __device__ __forceinline__ void init(const ConvGeom &geom, int n0, int group, int tid, int kend) {
        g = geom;
        rsrc = make_rsrc(g.x, g.x_bytes);
        k_end = kend;
        px.init(g, n0 + (tid % BN), group);
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
        const int KH = KHC > 0 ? KHC : g.KH;
        const int KW = KWC > 0 ? KWC : g.KW;
        const int KHW = KH * KW;
        const int kt = tid / BN;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int k = k0 + kt + i * KSTEP;
            const int c = k / KHW;
            const int rr = k - c * KHW;
            const int kh = rr / KW;
            const int kw = rr - kh * KW;
            const int ih = px.ih0 + kh;
            const int iw = px.iw0 + kw;
            const bool ok = px.valid && k < k_end && (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
            r[i] = buf_f32(rsrc, ok ? (px.base + ((uint32_t)c * g.H + ih) * g.W + iw) * 4u : kOOB);
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
        const int kt = tid / BN;
        const int n = tid % BN;
#pragma unroll
        for (int i = 0; i < NV; ++i) lds[(kt + i * KSTEP) * S + LdsPad<BN>::col(kt + i * KSTEP, n)] = r[i];
    }
};

// im2col gather, K in (kh, kw, c) order; needs Cg % BK == 0 so one BK slice is
// a single tap (kh, kw) over BK consecutive channels: one bounds test per
// thread per slice, then BK/KSTEP loads strided by one channel plane.
template <int BN, int BK>
struct Im2colTapLoader {
    static constexpr int S = LdsPad<BN>::stride;
    static constexpr int NV = BK * BN / kThreads;
    static constexpr int KSTEP = kThreads / BN;
    __amdgpu_buffer_rsrc_t rsrc;
    ConvGeom g;
    PixelOrigin px;
    uint32_t hw;
    float r[NV];
    // k0 of the previous fetch and its decomposition k_last = (kh * KW + kw) * Cg + c0
    // (wave-uniform): each loader copy sees k0 only grow, by a fixed step of one
    // or two slices, so the tap follows by carries instead of two integer
    // divisions per slice (k0 < KH * KW * Cg bounds the carries of a first fetch).
    int k_last, c0, kh, kw;

    __device__ __forceinline__ void init(const ConvGeom &geom, int n0, int group, int tid, int /*kend*/) {
        g = geom;
        rsrc = make_rsrc(g.x, g.x_bytes);
        hw = (uint32_t)(g.H * g.W);
        px.init(g, n0 + (tid % BN), group);
        k_last = c0 = kh = kw = 0;
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
        if (k0 < k_last) c0 = kh = kw = k_last = 0;
        c0 += k0 - k_last;
        while (c0 >= g.Cg) {
            c0 -= g.Cg;
            if (++kw == g.KW) {
                kw = 0;
                ++kh;
            }
        }
        k_last = k0;
        const int ih = px.ih0 + kh;
        const int iw = px.iw0 + kw;
        // taps past the window (fetches beyond the end of K) read zeros too
        const bool ok = px.valid && kh < g.KH && (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
        const uint32_t off0 = (px.base + (uint32_t)(c0 + tid / BN) * hw + (uint32_t)ih * g.W + iw) * 4u;
#pragma unroll
        for (int i = 0; i < NV; ++i) r[i] = buf_f32(rsrc, ok ? off0 + (uint32_t)(i * KSTEP) * hw * 4u : kOOB);
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
        const int kt = tid / BN;
        const int n = tid % BN;
#pragma unroll
        for (int i = 0; i < NV; ++i) lds[(kt + i * KSTEP) * S + LdsPad<BN>::col(kt + i * KSTEP, n)] = r[i];
    }
};

// 1x1 stride-1 unpadded convolution: im2col is the input itself, column j =
// (img, p) reads x[img][group*Cg + k][p]. With OH*OW a multiple of 4, four
// consecutive columns starting at a multiple of 4 lie in one image and one
// 16-byte aligned run, so each thread moves float4s exactly like KMajorLoader,
// with the image stride folded into a per-thread base computed once.
template <int BN, int BK>
struct Pointwise1x1Loader {
    static constexpr int S = LdsPad<BN>::stride;
    static constexpr int NV = (BK * BN / 4) / kThreads;
    static_assert(NV >= 1, "tile too small for 256 threads");
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t hw;
    uint32_t base[NV]; // element offset of (img, group*Cg, p) of this thread's columns; kOOB past ntot
    int k_end;
    f32x4 rv[NV];

    __device__ __forceinline__ void init(const ConvGeom &g, int n0, int group, int tid, int kend) {
        rsrc = make_rsrc(g.x, g.x_bytes);
        hw = (uint32_t)(g.OH * g.OW);
        k_end = kend;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = tid + i * kThreads;
            const int j = n0 + (c % (BN / 4)) * 4;
            const int img = j / (int)hw;
            const uint32_t p = (uint32_t)(j - img * (int)hw);
            base[i] = j < g.ntot ? ((uint32_t)img * g.C + (uint32_t)group * g.Cg) * hw + p : kOOB;
        }
    }
    __device__ __forceinline__ void fetch(int k0, int tid) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = tid + i * kThreads;
            const int k = k0 + c / (BN / 4);
            const bool ok = base[i] != kOOB && k < k_end;
            rv[i] = buf_f32x4(rsrc, ok ? (base[i] + (uint32_t)k * hw) * 4u : kOOB);
        }
    }
    __device__ __forceinline__ void commit(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = tid + i * kThreads;
            const int k = c / (BN / 4);
            *reinterpret_cast<f32x4 *>(lds + k * S + LdsPad<BN>::col(k, (c % (BN / 4)) * 4)) = rv[i];
        }
    }
};

// Output tile of this workgroup. Workgroups are dispatched round-robin over
// the 8 XCDs (each with its own L2), so consecutive block ids land on
// different XCDs. Remap so that each XCD walks a contiguous run of the tile
// space, M fastest: blocks sharing an L2 share the same input columns (the B
// operand, usually the larger one) and stream the weight rows in order.
// A bijection on [0, tiles_m * tiles_n) for each blockIdx.z.
__device__ __forceinline__ void xcd_tile(int tiles_m, int tiles_n, int &tm, int &tn) {
    constexpr int kXcds = 8;
    const int total = tiles_m * tiles_n;
    const int id = blockIdx.x + blockIdx.y * gridDim.x;
    const int xcd = id % kXcds;
    const int idx = id / kXcds;
    const int base = total / kXcds;
    const int rem = total % kXcds;
    const int t = xcd * base + min(xcd, rem) + idx;
    tm = t % tiles_m;
    tn = t / tiles_m;
}

// Reads all operand fragments of one LDS slice (issued together, so their
// latency overlaps the MFMAs that follow).
template <int BM, int BN, int BK>
__device__ __forceinline__ void load_fragments(const float *__restrict__ As, const float *__restrict__ Bs,
                                               float (&a)[BK / 2][WaveTiling<BM, BN>::TM],
                                               float (&b)[BK / 2][WaveTiling<BM, BN>::TN], int wm0, int wn0,
                                               int lane) {
    constexpr int SA = LdsPad<BM>::stride;
    constexpr int SB = LdsPad<BN>::stride;
    const int h = lane >> 5; // row parity of this half-wave's fetches
    const float *ap = As + h * SA;
    const float *bp = Bs + h * SB;
    int ac[WaveTiling<BM, BN>::TM], bc[WaveTiling<BM, BN>::TN];
#pragma unroll
    for (int i = 0; i < WaveTiling<BM, BN>::TM; ++i) ac[i] = LdsPad<BM>::col(h, wm0 + i * 32 + (lane & 31));
#pragma unroll
    for (int j = 0; j < WaveTiling<BM, BN>::TN; ++j) bc[j] = LdsPad<BN>::col(h, wn0 + j * 32 + (lane & 31));
#pragma unroll
    for (int q = 0; q < BK / 2; ++q) {
#pragma unroll
        for (int i = 0; i < WaveTiling<BM, BN>::TM; ++i) a[q][i] = ap[(2 * q) * SA + ac[i]];
#pragma unroll
        for (int j = 0; j < WaveTiling<BM, BN>::TN; ++j) b[q][j] = bp[(2 * q) * SB + bc[j]];
    }
}

template <int BM, int BN, int BK, int Q0, int Q1>
__device__ __forceinline__ void mfma_steps(const float (&a)[BK / 2][WaveTiling<BM, BN>::TM],
                                           const float (&b)[BK / 2][WaveTiling<BM, BN>::TN],
                                           f32x16 (&acc)[WaveTiling<BM, BN>::TM][WaveTiling<BM, BN>::TN]) {
#pragma unroll
    for (int q = Q0; q < Q1; ++q)
#pragma unroll
        for (int i = 0; i < WaveTiling<BM, BN>::TM; ++i)
#pragma unroll
            for (int j = 0; j < WaveTiling<BM, BN>::TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q][i], b[q][j], acc[i][j], 0, 0, 0);
}

// One pipelined slice: MFMAs of slice s (from LDS buffer `cur`), with the
// LDS write of slice s+1 (register stage `al/bl`) and the global fetch of
// slice s+3 (into the same, now free, register stage) between its halves.
// Both happen unconditionally: a fetch past the end of K reads through the
// operand's bounded buffer descriptor (zeros, or data the loop never
// consumes), so no branch hides the load count from the wait-count logic.
template <int BM, int BN, int BK, class AL, class BL>
__device__ __forceinline__ void pipelined_slice(AL &al, BL &bl, const float *As_cur, const float *Bs_cur,
                                                float *As_nxt, float *Bs_nxt,
                                                f32x16 (&acc)[WaveTiling<BM, BN>::TM][WaveTiling<BM, BN>::TN],
                                                int k_fetch, int tid, int lane, int wm0, int wn0) {
    float a[BK / 2][WaveTiling<BM, BN>::TM], b[BK / 2][WaveTiling<BM, BN>::TN];
    load_fragments<BM, BN, BK>(As_cur, Bs_cur, a, b, wm0, wn0, lane);
    __builtin_amdgcn_sched_barrier(0);
    mfma_steps<BM, BN, BK, 0, BK / 4>(a, b, acc);
    __builtin_amdgcn_sched_barrier(0);
    al.commit(As_nxt, tid);
    bl.commit(Bs_nxt, tid);
    __builtin_amdgcn_sched_barrier(0);
    al.fetch(k_fetch, tid);
    bl.fetch(k_fetch, tid);
    __builtin_amdgcn_sched_barrier(0);
    mfma_steps<BM, BN, BK, BK / 4, BK / 2>(a, b, acc);
    __syncthreads();
}

// The K loop shared by every MFMA GEMM kernel: BK slices through two LDS
// buffers and NS register stages (NS even). Slice j is fetched from global
// memory into register stage j % NS during slice j-1-NS, written to LDS buffer
// j % 2 during slice j-1 and consumed in slice j, so a global load has NS full
// slices of MFMA work to arrive. That distance is what keeps a lone workgroup
// per CU (small grids, split K, batch 1) from stalling on every slice: under
// load, HBM latency is several slices of 64x64 MFMA work. The LDS writes,
// address math and loads all overlap the matrix pipe; one barrier per slice.
// The steady-state loop is unrolled by NS so every stage is addressed
// statically. `al_init/bl_init` are loaders initialised for this tile; each
// stage is a copy of them. `init(acc)` sets the accumulators' start values;
// it runs right after the first slice's loads are issued, so loads it makes
// (a fused epilogue's bias and residual) overlap the prologue.
template <int BM, int BN, int BK, int NS, class AL, class BL, class Init>
__device__ __forceinline__ void gemm_mainloop(const AL &al_init, const BL &bl_init,
                                              float (*As)[BK * LdsPad<BM>::stride],
                                              float (*Bs)[BK * LdsPad<BN>::stride],
                                              f32x16 (&acc)[WaveTiling<BM, BN>::TM][WaveTiling<BM, BN>::TN],
                                              int k_begin, int nslices, int tid, int lane, int wm0, int wn0,
                                              const Init &init) {
    static_assert(NS >= 2 && NS % 2 == 0, "the LDS buffer of a slice is its parity: NS must be even");
    if (nslices <= 0) {
        init(acc);
        return;
    }
    AL al[NS];
    BL bl[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        al[i] = al_init;
        bl[i] = bl_init;
    }
    // prologue: slice 0 -> LDS 0; slices 1..NS -> register stage j % NS
    al[0].fetch(k_begin, tid);
    bl[0].fetch(k_begin, tid);
    init(acc);
    al[0].commit(As[0], tid);
    bl[0].commit(Bs[0], tid);
#pragma unroll
    for (int j = 1; j <= NS; ++j) {
        al[j % NS].fetch(k_begin + j * BK, tid);
        bl[j % NS].fetch(k_begin + j * BK, tid);
    }
    __syncthreads();
    int s = 0;
    for (; s + NS < nslices; s += NS) {
        // slice s+u reads LDS (s+u)%2 = u%2, commits slice s+u+1 from stage
        // (u+1)%NS and refills that stage with slice s+u+1+NS
#pragma unroll
        for (int u = 0; u < NS; ++u)
            pipelined_slice<BM, BN, BK>(al[(u + 1) % NS], bl[(u + 1) % NS], As[u % 2], Bs[u % 2], As[(u + 1) % 2],
                                        Bs[(u + 1) % 2], acc, k_begin + (s + u + 1 + NS) * BK, tid, lane, wm0, wn0);
    }
    // tail: r = nslices - s slices left, 1 <= r <= NS; the last one only computes
    const int r = nslices - s;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        if (u < r - 1) {
            pipelined_slice<BM, BN, BK>(al[(u + 1) % NS], bl[(u + 1) % NS], As[u % 2], Bs[u % 2], As[(u + 1) % 2],
                                        Bs[(u + 1) % 2], acc, k_begin + (s + u + 1 + NS) * BK, tid, lane, wm0, wn0);
        } else if (u == r - 1) {
            float a[BK / 2][WaveTiling<BM, BN>::TM], b[BK / 2][WaveTiling<BM, BN>::TN];
            load_fragments<BM, BN, BK>(As[u % 2], Bs[u % 2], a, b, wm0, wn0, lane);
            mfma_steps<BM, BN, BK, 0, BK / 2>(a, b, acc);
        }
    }
}

} // namespace spinn
