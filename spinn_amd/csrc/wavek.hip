// wavek.hip - fp32 MFMA GEMM for problems too small to fill the chip with
// 64 x 64 tiles (convolution layers at batch 1, the single Conv3x3+BN+ReLU
// layer, the Gemm sweep, fully-connected layers over a batch).
//
// One workgroup owns one TS x TS output tile (TS = 32, or 16 where 32-wide
// tiles still leave most CUs idle) and splits its K range over its KG waves. Each wave streams its operands from memory straight into MFMA
// operand registers - no LDS staging and no barrier in the K loop, two chunks
// of 32 k in flight - and the KG partial tiles are summed in a fixed order
// through LDS before the fused epilogue. This replaces, for these shapes,
// split K over workgroups followed by a separate reduction launch: one launch,
// deterministic, no workspace.
//
// v_mfma_f32_32x32x2f32 register layout: A operand lane l = A[l%32][k],
// B operand lane l = B[k][l%32], accumulator element r of lane l =
// D[8*(r/4) + 4*(l/32) + r%4][l%32]; the two half-waves h = l/32 supply the
// two k of a step. v_mfma_f32_16x16x4f32: A lane l = A[l%16][k], B lane l =
// B[k][l%16], accumulator element r of lane l = D[4*(l/16) + r][l%16]; the four
// lane groups h = l/16 supply the four k of a step. A block of 4 * groups k
// (8 or 16) is 4 steps q, and lane group h of step q takes k = 4h + q: a
// k-contiguous operand is then one 16-byte load per lane per block. (Which k
// feeds which step and group does not change the sum's terms; A and B use the
// same assignment.)
#include "mfma_core.h"
#include "spinn_hip_internal.h"
#include <type_traits>

namespace spinn {

namespace {

// The MFMA shape of a TS x TS tile: lane groups, k per block (4 steps), and
// the accumulator.
template <int TS>
struct WkShape;
template <>
struct WkShape<32> {
    using Acc = f32x16;
    static constexpr int kAcc = 16;
    static constexpr int kBlock = 8; // 2 lane groups x 4 steps
    __device__ static int group(int lane) { return lane >> 5; }
    __device__ static int col(int lane) { return lane & 31; }
    __device__ static int row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
    __device__ static Acc mfma(float a, float b, const Acc &c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};
template <>
struct WkShape<16> {
    using Acc = f32x4;
    static constexpr int kAcc = 4;
    static constexpr int kBlock = 16; // 4 lane groups x 4 steps
    __device__ static int group(int lane) { return lane >> 4; }
    __device__ static int col(int lane) { return lane & 15; }
    __device__ static int row(int r, int lane) { return 4 * (lane >> 4) + r; }
    __device__ static Acc mfma(float a, float b, const Acc &c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};
// k per chunk: 4 blocks
template <int TS>
constexpr int wk_chunk() { return 4 * WkShape<TS>::kBlock; }

// ---- operand fetchers: one k block, the lane's 4 values (steps q) of lane group h ----

// Source [K][ld] with the tile index contiguous: v[q] = src[(k0 + 4h + q) * ld + t].
struct WkTContig {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t ld, t;
    bool t_ok;
    int k_end;
    __device__ __forceinline__ void init(const float *base, uint32_t bytes, uint32_t ld_, int t_, int t_total,
                                         int kend) {
        rsrc = make_rsrc(base, bytes);
        ld = ld_;
        t = (uint32_t)t_;
        t_ok = t_ < t_total;
        k_end = kend;
    }
    __device__ __forceinline__ void fetch(int k0, int h, float (&v)[4]) const {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = k0 + 4 * h + q;
            v[q] = buf_f32(rsrc, (t_ok && k < k_end) ? ((uint32_t)k * ld + t) * 4u : kOOB);
        }
    }
};

// Source [T][ld] with k contiguous: v = src[t * ld + k0 + 4h .. +3]; VEC: one
// 16-byte load (ld % 4 == 0, aligned base, k_end % 4 == 0). The lane's row
// offset is computed once, with the row test folded in (kOOB for rows past
// t_total: adding a k offset below 2^31 keeps it out of range without
// wrapping); a block then costs one add and the K-end test.
template <bool VEC>
struct WkKContig {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t row, vrow;
    bool t_ok;
    int k_end;
    __device__ __forceinline__ void init(const float *base, uint32_t bytes, uint32_t ld, int t, int t_total,
                                         int kend) {
        rsrc = make_rsrc(base, bytes);
        t_ok = t < t_total;
        row = t_ok ? (uint32_t)t * ld : 0u;
        vrow = t_ok ? row * 4u : kOOB;
        k_end = kend;
    }
    __device__ __forceinline__ void fetch(int k0, int h, float (&v)[4]) const {
        const int k = k0 + 4 * h;
        if constexpr (VEC) {
            const f32x4 r = buf_f32x4(rsrc, k < k_end ? vrow + (uint32_t)k * 4u : kOOB);
            v[0] = r[0];
            v[1] = r[1];
            v[2] = r[2];
            v[3] = r[3];
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v[q] = buf_f32(rsrc, (t_ok && k + q < k_end) ? (row + (uint32_t)(k + q)) * 4u : kOOB);
        }
    }
};

// Implicit-GEMM B operand, 1x1 stride-1 unpadded conv: column n = (img, p)
// reads x[img][g*Cg + k][p]. The lane's pixel is a byte offset with the column
// test folded in (kOOB past ntot: adding a channel offset below 2^31 keeps it
// out of range without wrapping), so a load costs one add. K is a multiple of
// the k block (the caller's condition; the per-wave ranges are block multiples),
// so a block is wholly inside or past the wave's K end and the test is a
// wave-uniform choice of descriptor, one of size 0 past the end.
struct WkPointwise {
    __amdgpu_buffer_rsrc_t rsrc, rnone;
    uint32_t vbase, hw4;
    int k_end;
    __device__ __forceinline__ void init(const ConvGeom &g, int n, int group, int kend) {
        rsrc = make_rsrc(g.x, g.x_bytes);
        rnone = make_rsrc(g.x, 0u);
        const uint32_t hw = (uint32_t)(g.OH * g.OW);
        hw4 = hw * 4u;
        const bool ok = n < g.ntot;
        const int nn = ok ? n : 0;
        const int img = nn / (int)hw;
        vbase = ok ? (((uint32_t)img * g.C + (uint32_t)group * g.Cg) * hw + (uint32_t)(nn - img * (int)hw)) * 4u
                   : kOOB;
        k_end = kend;
    }
    __device__ __forceinline__ void fetch(int k0, int h, float (&v)[4]) const {
        const __amdgpu_buffer_rsrc_t r = k0 < k_end ? rsrc : rnone;
        const uint32_t off = vbase + (uint32_t)(k0 + 4 * h) * hw4;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = buf_f32(r, off + (uint32_t)q * hw4);
    }
};

// Implicit-GEMM B operand, K in (kh, kw, c) order with Cg % 16 == 0: a block
// of 8 or 16 k lies in one tap, so one bounds test per block. A wave fetches
// its blocks in increasing k, one block at a time: the loader keeps the next
// block's (kh, kw, c) position and steps it, instead of dividing k by Cg and
// KW for every block. Each lane keeps the byte offset of its pixel's current
// tap at channel 4h, or kOOB where the tap falls outside the image (adding a
// channel offset, below 2^31, keeps it out of range without wrapping); the
// channel offset of a block is wave-uniform, and a block at or past the K end
// reads through a descriptor of size 0. A block's four loads then cost one add
// each, and only a change of tap recomputes the lane's offset.
struct WkTap {
    __amdgpu_buffer_rsrc_t rsrc, rnone;
    PixelOrigin px;
    uint32_t hw, hw4, lane_c; // lane_c: the lane's channel offset 4h * hw
    int Cg, KW, KH, H, W;
    int k_end;
    int blk, c_cur, kh_cur, kw_cur; // block size and the next block's position
    uint32_t vtap;                  // byte offset of (pixel, current tap, channel 4h), or kOOB
    __device__ __forceinline__ void init(const ConvGeom &g, int n, int group, int kend) {
        rsrc = make_rsrc(g.x, g.x_bytes);
        rnone = make_rsrc(g.x, 0u);
        px.init(g, n, group);
        hw = (uint32_t)(g.H * g.W);
        hw4 = hw * 4u;
        Cg = g.Cg;
        KW = g.KW;
        KH = g.KH;
        H = g.H;
        W = g.W;
        k_end = kend;
    }
    __device__ __forceinline__ void set_tap() {
        const int ih = px.ih0 + kh_cur;
        const int iw = px.iw0 + kw_cur;
        const bool ok = px.valid && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
        vtap = ok ? (px.base + lane_c + (uint32_t)ih * W + iw) * 4u : kOOB;
    }
    // First block at k = kb (a multiple of `block`), blocks of `block` k; h: the lane's group.
    __device__ __forceinline__ void start(int kb, int block, int h) {
        blk = block;
        lane_c = (uint32_t)(4 * h) * hw;
        const int tap = kb / Cg;
        c_cur = kb - tap * Cg;
        kh_cur = tap / KW;
        kw_cur = tap - kh_cur * KW;
        set_tap();
    }
    // The block at k0, which is the block after the previous call's.
    __device__ __forceinline__ void fetch(int k0, int, float (&v)[4]) {
        const __amdgpu_buffer_rsrc_t r = k0 < k_end ? rsrc : rnone;
        const uint32_t c_off = (uint32_t)c_cur * hw4;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = buf_f32(r, vtap + c_off + (uint32_t)q * hw4);
        c_cur += blk;
        if (c_cur >= Cg) {
            c_cur = 0;
            if (++kw_cur == KW) {
                kw_cur = 0;
                ++kh_cur;
            }
            set_tap();
        }
    }
};

// Implicit-GEMM B operand, K in the reference's (c, kh, kw) im2col order
// (SPINN/run_time/ops/conv/conv2d.c:58-76), any shape; compile-time KH, KW
// when given (0 = runtime).
template <int KHC, int KWC>
struct WkGather {
    __amdgpu_buffer_rsrc_t rsrc;
    PixelOrigin px;
    int KH, KW, H, W;
    int k_end;
    __device__ __forceinline__ void init(const ConvGeom &g, int n, int group, int kend) {
        rsrc = make_rsrc(g.x, g.x_bytes);
        px.init(g, n, group);
        KH = KHC > 0 ? KHC : g.KH;
        KW = KWC > 0 ? KWC : g.KW;
        H = g.H;
        W = g.W;
        k_end = kend;
    }
    __device__ __forceinline__ void fetch(int k0, int h, float (&v)[4]) const {
        const int khw = KH * KW;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = k0 + 4 * h + q;
            const int c = k / khw;
            const int r = k - c * khw;
            const int kh = r / KW;
            const int kw = r - kh * KW;
            const int ih = px.ih0 + kh;
            const int iw = px.iw0 + kw;
            const bool ok = px.valid && k < k_end && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            v[q] = buf_f32(rsrc, ok ? (px.base + ((uint32_t)c * H + ih) * W + iw) * 4u : kOOB);
        }
    }
};

// ---- the K loop of one wave and the cross-wave sum ----

template <int TS, class AF, class BF>
__device__ __forceinline__ void wk_fetch(const AF &af, BF &bf, int k0, int h, float (&a)[4][4],
                                         float (&b)[4][4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        af.fetch(k0 + WkShape<TS>::kBlock * u, h, a[u]);
        bf.fetch(k0 + WkShape<TS>::kBlock * u, h, b[u]);
    }
}

template <int TS>
__device__ __forceinline__ void wk_mfma(const float (&a)[4][4], const float (&b)[4][4],
                                        typename WkShape<TS>::Acc &acc) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = WkShape<TS>::mfma(a[u][q], b[u][q], acc);
}

// The first `blocks` (wave-uniform) blocks of a chunk: the MFMAs of a chunk's
// all-zero tail blocks are skipped.
template <int TS>
__device__ __forceinline__ void wk_mfma_part(const float (&a)[4][4], const float (&b)[4][4], int blocks,
                                             typename WkShape<TS>::Acc &acc) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (u < blocks)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = WkShape<TS>::mfma(a[u][q], b[u][q], acc);
}

// acc = sum over k in [kb, ke) of A[m][k] B[k][n] for this lane's accumulator
// elements, with NB chunks of 4 blocks in flight (NB = 2 or 4): while chunk c
// computes, chunks c+1 .. c+NB-1 are loading. A lone wave on its SIMD (small
// grids) needs the deeper ring: one chunk is 16 MFMAs, about 0.2-0.4 us, well
// under the memory latency under load. Fetchers read zero at and past their
// k_end (= ke), so chunks past the end need no branch; every fetch has a use
// on every path, so none can be sunk below the MFMAs it is meant to overlap.
template <int TS, int NB, class AF, class BF>
__device__ __forceinline__ void wk_accumulate(const AF &af, BF &bf, int kb, int ke, int h,
                                              typename WkShape<TS>::Acc &acc) {
    static_assert(NB == 2 || NB == 4, "ring of 2 or 4 chunks");
    constexpr int kChunk = wk_chunk<TS>();
    constexpr int kBlock = WkShape<TS>::kBlock;
#pragma unroll
    for (int r = 0; r < WkShape<TS>::kAcc; ++r) acc[r] = 0.f;
    if (kb >= ke) return;
    const int nch = (ke - kb + kChunk - 1) / kChunk;
    float a[NB][4][4], b[NB][4][4];
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) wk_fetch<TS>(af, bf, kb + i * kChunk, h, a[i], b[i]);
    int c = 0;
    for (; c + NB <= nch; c += NB) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            // slot (i + NB - 1) % NB receives chunk c + i + NB - 1 while slot i computes chunk c + i
            wk_fetch<TS>(af, bf, kb + (c + i + NB - 1) * kChunk, h, a[(i + NB - 1) % NB], b[(i + NB - 1) % NB]);
            wk_mfma<TS>(a[i], b[i], acc);
        }
    }
    // 0 .. NB-1 chunks left, in slots 0 .. NB-2; the last one may hold fewer than 4 blocks
#pragma unroll
    for (int i = 0; i < NB - 1; ++i)
        if (c + i < nch) wk_mfma_part<TS>(a[i], b[i], (ke - kb - (c + i) * kChunk + kBlock - 1) / kBlock, acc);
}

// Per-wave K range: KG slices of kq (a multiple of the k block).
__device__ __forceinline__ void wk_range(int K, int kq, int wave, int &kb, int &ke) {
    kb = min(K, wave * kq);
    ke = min(K, kb + kq);
}

// Outputs of the tile per thread in the cross-wave sum: output i of a thread is
// element e = threadIdx.x + 64 KG i (e < TS * TS) of the wave-order layout.
template <int TS, int KG>
constexpr int wk_outs() { return (TS * TS + 64 * KG - 1) / (64 * KG); }

// Call `f(i, m_local, n_local)` for each output i of this thread.
template <int TS, int KG, class F>
__device__ __forceinline__ void wk_for_outputs(const F &f) {
#pragma unroll
    for (int i = 0; i < wk_outs<TS, KG>(); ++i) {
        const int e = threadIdx.x + 64 * KG * i;
        if (e < TS * TS) f(i, WkShape<TS>::row(e >> 6, e & 63), WkShape<TS>::col(e & 63));
    }
}

// Sum the KG partial tiles in wave order and hand each output (m, n) to
// `store(i, m_local, n_local, v)`; consecutive threads take consecutive columns.
// The kernels load what the epilogue adds (bias, residual, C) for the same
// outputs i before their K loop, so those loads are in flight during it
// instead of one round trip per output after the sum.
template <int TS, int KG, class Store>
__device__ __forceinline__ void wk_reduce_store(const typename WkShape<TS>::Acc &acc,
                                                float (*red)[WkShape<TS>::kAcc][64], const Store &store) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < WkShape<TS>::kAcc; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < wk_outs<TS, KG>(); ++i) {
        const int e = threadIdx.x + 64 * KG * i;
        if (e >= TS * TS) break;
        const int r = e >> 6;
        const int l = e & 63;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < KG; ++w) v += red[w][r][l];
        store(i, WkShape<TS>::row(r, l), WkShape<TS>::col(l), v);
    }
}

// ---- kernels ----

struct WkConvArgs {
    const float *wpk; // packed W^T [group][K][ldw], or weights [group][OCg][K] with K contiguous
    int64_t wpk_group_stride;
    int ldw;
    int M, K; // per group
    int kq;   // K per wave
    ConvGeom geom;
    float *__restrict__ y;
    const float *__restrict__ bias;
    const float *__restrict__ res;
    int act;
    int OC, OHW;
};

// AF: WkTContig over the packed W^T [K][ldw], or WkKContig<true> over the raw
// weights W [OC][K] (K in (c, kh, kw) order) or the packing's tap-ordered
// [OCg][K] copy (16-byte loads along k).
template <int TS, int KG, int NB, class AF, class BF>
__global__ __launch_bounds__(64 * KG) void wavek_conv_kernel(WkConvArgs a) {
    using S = WkShape<TS>;
    __shared__ float red[KG][S::kAcc][64];
    const int lane = threadIdx.x & 63;
    // wave-uniform: the K range and the tap / channel split of every block are scalar work
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = S::group(lane);
    int tm, tn;
    xcd_tile(gridDim.y, gridDim.x, tm, tn);
    const int m0 = tm * TS, n0 = tn * TS;
    const int group = blockIdx.z;
    int kb, ke;
    wk_range(a.K, a.kq, wave, kb, ke);
    AF af;
    if constexpr (std::is_same<AF, WkTContig>::value)
        af.init(a.wpk + group * a.wpk_group_stride, (uint32_t)a.K * (uint32_t)a.ldw * 4u, (uint32_t)a.ldw,
                m0 + S::col(lane), a.M, ke);
    else
        af.init(a.wpk + group * a.wpk_group_stride, (uint32_t)a.M * (uint32_t)a.K * 4u, (uint32_t)a.K,
                m0 + S::col(lane), a.M, ke);
    BF bf;
    bf.init(a.geom, n0 + S::col(lane), group, ke);
    if constexpr (std::is_same<BF, WkTap>::value) bf.start(kb, S::kBlock, h);
    // output index, bias and residual of each of this thread's outputs (idx < 0: outside the
    // problem; y is at most 2 GiB, so an element index fits 32 bits)
    const int ntot = a.geom.ntot;
    constexpr int NO = wk_outs<TS, KG>();
    int oidx[NO];
    float ob[NO], orr[NO];
    wk_for_outputs<TS, KG>([&](int i, int ml, int nl) {
        const int m = m0 + ml, n = n0 + nl;
        oidx[i] = -1;
        ob[i] = orr[i] = 0.f;
        if (m >= a.M || n >= ntot) return;
        const int img = n / a.OHW;
        const int p = n - img * a.OHW;
        const int oc = group * a.M + m;
        oidx[i] = (int)(((int64_t)img * a.OC + oc) * a.OHW + p);
        if (a.bias) ob[i] = a.bias[oc];
        if (a.res) orr[i] = a.res[oidx[i]];
    });
    typename S::Acc acc;
    wk_accumulate<TS, NB>(af, bf, kb, ke, h, acc);
    wk_reduce_store<TS, KG>(acc, red, [&](int i, int, int, float v) {
        if (oidx[i] < 0) return;
        // the reference's order: acc + bias, then + residual (gemm_kernel.c:316-338)
        if (a.bias) v += ob[i];
        if (a.res) v += orr[i];
        a.y[oidx[i]] = apply_act(v, a.act);
    });
}

struct WkGemmArgs {
    const float *__restrict__ a;
    const float *__restrict__ b;
    const float *__restrict__ c;
    int64_t lda, ldb;
    int64_t stride_a, stride_b, stride_y;
    int M, N, K, kq;
    int c_mode;
    float alpha, beta;
    float *__restrict__ y;
};

template <int TS, int KG, int NB, class AF, class BF>
__global__ __launch_bounds__(64 * KG) void wavek_gemm_kernel(WkGemmArgs a) {
    using S = WkShape<TS>;
    __shared__ float red[KG][S::kAcc][64];
    const int lane = threadIdx.x & 63;
    // wave-uniform: the K range and the tap / channel split of every block are scalar work
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = S::group(lane);
    int tm, tn;
    xcd_tile(gridDim.y, gridDim.x, tm, tn);
    const int m0 = tm * TS, n0 = tn * TS;
    const int batch = blockIdx.z;
    int kb, ke;
    wk_range(a.K, a.kq, wave, kb, ke);
    AF af;
    BF bf;
    // A rows are m: k-major [K][lda] when transposed, else [M][lda] with k contiguous
    const float *abase = a.a + batch * a.stride_a;
    const float *bbase = a.b + batch * a.stride_b;
    if constexpr (std::is_same<AF, WkTContig>::value)
        af.init(abase, (uint32_t)(a.K * a.lda * 4), (uint32_t)a.lda, m0 + S::col(lane), a.M, ke);
    else
        af.init(abase, (uint32_t)(a.M * a.lda * 4), (uint32_t)a.lda, m0 + S::col(lane), a.M, ke);
    // B columns are n: k-major [K][ldb] when not transposed, else [N][ldb] with k contiguous
    if constexpr (std::is_same<BF, WkTContig>::value)
        bf.init(bbase, (uint32_t)(a.K * a.ldb * 4), (uint32_t)a.ldb, n0 + S::col(lane), a.N, ke);
    else
        bf.init(bbase, (uint32_t)(a.N * a.ldb * 4), (uint32_t)a.ldb, n0 + S::col(lane), a.N, ke);
    // C value of each of this thread's outputs, loaded before the K loop
    constexpr int NO = wk_outs<TS, KG>();
    float oc_[NO];
    wk_for_outputs<TS, KG>([&](int i, int ml, int nl) {
        const int m = m0 + ml, n = n0 + nl;
        oc_[i] = 0.f;
        if (m >= a.M || n >= a.N) return;
        if (a.c_mode == 1) oc_[i] = a.c[n];
        else if (a.c_mode == 2) oc_[i] = a.c[(int64_t)m * a.N + n];
    });
    typename S::Acc acc;
    wk_accumulate<TS, NB>(af, bf, kb, ke, h, acc);
    wk_reduce_store<TS, KG>(acc, red, [&](int i, int ml, int nl, float v) {
        const int m = m0 + ml, n = n0 + nl;
        if (m >= a.M || n >= a.N) return;
        v *= a.alpha;
        if (a.c_mode == 1 || a.c_mode == 2) v += a.beta * oc_[i];
        a.y[batch * a.stride_y + (int64_t)m * a.N + n] = v;
    });
}

// Waves per workgroup: doubled while the grid has fewer than 2048 waves and
// each wave keeps at least one chunk, up to 8 (512 threads: more would cap a
// lane at 128 registers, below what the gather loaders hold).
int wavek_waves(int64_t tiles, int K, int chunk) {
    int kg = 1;
    while (kg < 8 && tiles * kg < 2048 && K / (2 * kg) >= chunk) kg *= 2;
    return kg;
}

int wavek_kq(int K, int kg, int block) { return ((K + kg - 1) / kg + block - 1) / block * block; }

template <int TS, int NB, class AF, class BF>
int launch_wk_conv_nb(const WkConvArgs &a, int kg, dim3 grid, hipStream_t st) {
    switch (kg) {
    case 1: hipLaunchKernelGGL((wavek_conv_kernel<TS, 1, NB, AF, BF>), grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((wavek_conv_kernel<TS, 2, NB, AF, BF>), grid, dim3(128), 0, st, a); break;
    case 4: hipLaunchKernelGGL((wavek_conv_kernel<TS, 4, NB, AF, BF>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((wavek_conv_kernel<TS, 8, NB, AF, BF>), grid, dim3(512), 0, st, a); break;
    }
    return check_launch();
}

// Waves with at most 4 chunks use the 2-deep ring, longer ones the 4-deep one:
// the deep ring issues 4 chunks of loads before a wave's first MFMA, which for
// a short K range only delays it (measured on the 1x64x56x56 3x3 layer, 72 k
// per wave: 8.25 -> 7.85 us).
bool wk_deep(int kq, int chunk) { return kq > 4 * chunk; }

template <class AF, class BF>
int launch_wk_conv(const WkConvArgs &a, int ts, int kg, dim3 grid, hipStream_t st) {
    if (ts == 16)
        return wk_deep(a.kq, wk_chunk<16>()) ? launch_wk_conv_nb<16, 4, AF, BF>(a, kg, grid, st)
                                             : launch_wk_conv_nb<16, 2, AF, BF>(a, kg, grid, st);
    return wk_deep(a.kq, wk_chunk<32>()) ? launch_wk_conv_nb<32, 4, AF, BF>(a, kg, grid, st)
                                         : launch_wk_conv_nb<32, 2, AF, BF>(a, kg, grid, st);
}

template <int TS, int NB, class AF, class BF>
int launch_wk_gemm_nb(const WkGemmArgs &a, int kg, dim3 grid, hipStream_t st) {
    switch (kg) {
    case 1: hipLaunchKernelGGL((wavek_gemm_kernel<TS, 1, NB, AF, BF>), grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((wavek_gemm_kernel<TS, 2, NB, AF, BF>), grid, dim3(128), 0, st, a); break;
    case 4: hipLaunchKernelGGL((wavek_gemm_kernel<TS, 4, NB, AF, BF>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((wavek_gemm_kernel<TS, 8, NB, AF, BF>), grid, dim3(512), 0, st, a); break;
    }
    return check_launch();
}

template <class AF, class BF>
int launch_wk_gemm(const WkGemmArgs &a, int ts, int kg, dim3 grid, hipStream_t st) {
    if (ts == 16)
        return wk_deep(a.kq, wk_chunk<16>()) ? launch_wk_gemm_nb<16, 4, AF, BF>(a, kg, grid, st)
                                             : launch_wk_gemm_nb<16, 2, AF, BF>(a, kg, grid, st);
    return wk_deep(a.kq, wk_chunk<32>()) ? launch_wk_gemm_nb<32, 4, AF, BF>(a, kg, grid, st)
                                         : launch_wk_gemm_nb<32, 2, AF, BF>(a, kg, grid, st);
}

} // namespace

int wavek_conv(const SpinnHipConvDesc *d, int ts, const float *x, const float *w, const float *packed,
               const float *bias, const float *res, float *y, hipStream_t st) {
    WkConvArgs a{};
    const int OCg = d->oc / d->group;
    const int Cg = d->c / d->group;
    a.ldw = (OCg + 3) / 4 * 4;
    a.M = OCg;
    a.K = Cg * d->kh * d->kw;
    // The raw weights W [OC][K] give 16-byte loads along k (a quarter of the load
    // instructions of the packed layout's one-float-per-k loads) when K is a multiple
    // of 4 and W is 16-byte aligned; the B gather then follows W's (c, kh, kw) order.
    const bool pointwise = d->kh == 1 && d->kw == 1 && d->sh == 1 && d->sw == 1 && d->ph == 0 && d->pw == 0 &&
                           d->oh == d->h && d->ow == d->w;
    // WkPointwise tests the K end once per k block: K a multiple of the block
    // (every wave's range is a multiple of it); other 1x1 shapes take WkGather<1, 1>.
    const bool pw_blocks = pointwise && a.K % (ts == 16 ? WkShape<16>::kBlock : WkShape<32>::kBlock) == 0;
    // Raw weights need the B gather in (c, kh, kw) order, whose per-element index
    // arithmetic costs more than the 16-byte A loads save for windows larger than 1x1
    // when the packed layout is tap-ordered (16-channel multiples): there the packed
    // W^T and the one-test-per-block tap gather are used.
    const bool raw = w && a.K % 4 == 0 && ((uintptr_t)w & 15u) == 0 && (pointwise || Cg % kBK != 0);
    // Tap-ordered windows read the packing's k-contiguous copy [OCg][K] the same way.
    const float *kcopy = raw ? nullptr : igemm_kcopy(d, packed);
    const bool tap_k = kcopy && ((uintptr_t)kcopy & 15u) == 0;
    a.wpk = raw ? w : (tap_k ? kcopy : packed);
    a.wpk_group_stride = (raw || tap_k) ? (int64_t)OCg * a.K : (int64_t)a.K * a.ldw;
    if (!a.wpk) return SPINN_HIP_EINVAL;
    const uint64_t x_bytes = (uint64_t)d->n * d->c * d->h * d->w * sizeof(float);
    const uint64_t w_bytes = (uint64_t)d->group * a.K * ((raw || tap_k) ? OCg : a.ldw) * sizeof(float);
    const uint64_t y_bytes = (uint64_t)d->n * d->oc * d->oh * d->ow * sizeof(float);
    if (x_bytes > kMaxOperandBytes || w_bytes > kMaxOperandBytes || y_bytes > kMaxOperandBytes)
        return SPINN_HIP_EUNSUPPORTED;
    a.geom = ConvGeom{x, (uint32_t)x_bytes, d->c, d->h, d->w, Cg, d->oh, d->ow, d->kh, d->kw,
                      d->sh, d->sw, d->ph, d->pw, d->n * d->oh * d->ow};
    a.y = y;
    a.bias = bias;
    a.res = res;
    a.act = d->act;
    a.OC = d->oc;
    a.OHW = d->oh * d->ow;
    const dim3 grid((a.geom.ntot + ts - 1) / ts, (a.M + ts - 1) / ts, d->group);
    const int kg = wavek_waves((int64_t)grid.x * grid.y * grid.z, a.K, ts == 16 ? wk_chunk<16>() : wk_chunk<32>());
    a.kq = wavek_kq(a.K, kg, ts == 16 ? WkShape<16>::kBlock : WkShape<32>::kBlock);
    if (raw) {
        using RA = WkKContig<true>;
        if (pw_blocks) return launch_wk_conv<RA, WkPointwise>(a, ts, kg, grid, st);
        if (d->kh == 3 && d->kw == 3) return launch_wk_conv<RA, WkGather<3, 3>>(a, ts, kg, grid, st);
        if (d->kh == 7 && d->kw == 7) return launch_wk_conv<RA, WkGather<7, 7>>(a, ts, kg, grid, st);
        if (d->kh == 1 && d->kw == 1) return launch_wk_conv<RA, WkGather<1, 1>>(a, ts, kg, grid, st);
        return launch_wk_conv<RA, WkGather<0, 0>>(a, ts, kg, grid, st);
    }
    if (tap_k) return launch_wk_conv<WkKContig<true>, WkTap>(a, ts, kg, grid, st);
    if (!packed) return SPINN_HIP_EINVAL;
    if (pw_blocks) return launch_wk_conv<WkTContig, WkPointwise>(a, ts, kg, grid, st);
    if (Cg % kBK == 0) return launch_wk_conv<WkTContig, WkTap>(a, ts, kg, grid, st); // the pack's tap order
    if (d->kh == 3 && d->kw == 3) return launch_wk_conv<WkTContig, WkGather<3, 3>>(a, ts, kg, grid, st);
    if (d->kh == 7 && d->kw == 7) return launch_wk_conv<WkTContig, WkGather<7, 7>>(a, ts, kg, grid, st);
    if (d->kh == 1 && d->kw == 1) return launch_wk_conv<WkTContig, WkGather<1, 1>>(a, ts, kg, grid, st);
    return launch_wk_conv<WkTContig, WkGather<0, 0>>(a, ts, kg, grid, st);
}

int wavek_gemm(const SpinnHipGemmDesc *d, int ts, const float *A, const float *B, const float *C, float *Y,
               hipStream_t st) {
    WkGemmArgs a{};
    a.a = A;
    a.b = B;
    a.c = C;
    a.M = d->m;
    a.N = d->n;
    a.K = d->k;
    a.lda = d->trans_a ? d->m : d->k;
    a.ldb = d->trans_b ? d->k : d->n;
    const int batch = d->batch > 0 ? d->batch : 1;
    a.stride_a = d->stride_a;
    a.stride_b = d->stride_b;
    a.stride_y = d->stride_y;
    a.c_mode = C ? d->c_mode : 0;
    a.alpha = d->alpha;
    a.beta = d->beta;
    a.y = Y;
    const uint64_t a_bytes = (uint64_t)d->m * d->k * sizeof(float);
    const uint64_t b_bytes = (uint64_t)d->n * d->k * sizeof(float);
    if (a_bytes > kMaxOperandBytes || b_bytes > kMaxOperandBytes) return SPINN_HIP_EUNSUPPORTED;
    const dim3 grid((d->n + ts - 1) / ts, (d->m + ts - 1) / ts, batch);
    const int kg = wavek_waves((int64_t)grid.x * grid.y * grid.z, d->k, ts == 16 ? wk_chunk<16>() : wk_chunk<32>());
    a.kq = wavek_kq(d->k, kg, ts == 16 ? WkShape<16>::kBlock : WkShape<32>::kBlock);
    // 16-byte loads along k need 4-aligned rows in every batch entry and a K that is a multiple of 4
    const bool va = ((uintptr_t)A & 15u) == 0 && a.lda % 4 == 0 && d->k % 4 == 0 &&
                    (batch == 1 || d->stride_a % 4 == 0);
    const bool vb = ((uintptr_t)B & 15u) == 0 && a.ldb % 4 == 0 && d->k % 4 == 0 &&
                    (batch == 1 || d->stride_b % 4 == 0);
    if (d->trans_a) {
        if (d->trans_b)
            return vb ? launch_wk_gemm<WkTContig, WkKContig<true>>(a, ts, kg, grid, st)
                      : launch_wk_gemm<WkTContig, WkKContig<false>>(a, ts, kg, grid, st);
        return launch_wk_gemm<WkTContig, WkTContig>(a, ts, kg, grid, st);
    }
    if (d->trans_b) {
        if (va && vb) return launch_wk_gemm<WkKContig<true>, WkKContig<true>>(a, ts, kg, grid, st);
        if (va) return launch_wk_gemm<WkKContig<true>, WkKContig<false>>(a, ts, kg, grid, st);
        if (vb) return launch_wk_gemm<WkKContig<false>, WkKContig<true>>(a, ts, kg, grid, st);
        return launch_wk_gemm<WkKContig<false>, WkKContig<false>>(a, ts, kg, grid, st);
    }
    return va ? launch_wk_gemm<WkKContig<true>, WkTContig>(a, ts, kg, grid, st)
              : launch_wk_gemm<WkKContig<false>, WkTContig>(a, ts, kg, grid, st);
}

} // namespace spinn
