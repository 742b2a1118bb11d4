// gemm.hip - Gemm / MatMul on the fp32 MFMA tile engine.
//
// y[b] = alpha * op(A[b]) op(B[b]) + beta * C, row-major, any transpose
// combination: each operand is staged k-major in LDS by the loader matching
// its memory order (16-byte loads when rows are aligned), so a transposed B
// (the usual Gemm weight layout, transB=1) is read in place instead of being
// transposed into a temporary on every call (SPINN/run_time/ops/mm/gemm.c:50-59).
// Small grids split K over blockIdx.z with a deterministic reduction.
#include "mfma_core.h"
#include "spinn_hip_internal.h"
#include <type_traits>

namespace spinn {

// ---------------------------------------------------------------------------
// Gemm
// ---------------------------------------------------------------------------
struct GemmKArgs {
    const float *__restrict__ a;
    const float *__restrict__ b;
    const float *__restrict__ c;
    int64_t lda, ldb;
    int64_t stride_a, stride_b, stride_y;
    int M, N, K;
    int c_mode;
    float alpha, beta;
    float *__restrict__ y;
    float *__restrict__ ws;
    int k_chunk;
};

template <int BM, int BN, int BK, class ALoader, class BLoader, bool SPLIT>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(GemmKArgs a) {
    using WT = WaveTiling<BM, BN>;
    constexpr int SA = LdsPad<BM>::stride;
    constexpr int SB = LdsPad<BN>::stride;
    __shared__ __attribute__((aligned(16))) float As[2][BK * SA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = WT::origin_m(wave);
    const int wn0 = WT::origin_n(wave);
    int tile_m, tile_n;
    xcd_tile(gridDim.y, gridDim.x, tile_m, tile_n);
    const int n0 = tile_n * BN;
    const int m0 = tile_m * BM;
    const int z = blockIdx.z;
    const int batch = SPLIT ? 0 : z;
    const int k_begin = SPLIT ? z * a.k_chunk : 0;
    const int k_end = SPLIT ? min(a.K, k_begin + a.k_chunk) : a.K;

    ALoader al;
    BLoader bl;
    // A tile rows are m: KMajor source a[k*lda + m] (K rows), RowK source a[m*lda + k] (M rows).
    const float *abase = a.a + batch * a.stride_a;
    const float *bbase = a.b + batch * a.stride_b;
    if constexpr (ALoader::kIsKMajor) {
        al.init(abase, (uint32_t)(a.K * a.lda * 4), (uint32_t)a.lda, m0, a.M);
    } else {
        al.init(abase, (uint32_t)(a.M * a.lda * 4), (uint32_t)a.lda, m0, a.M, k_end);
    }
    if constexpr (BLoader::kIsKMajor) {
        bl.init(bbase, (uint32_t)(a.K * a.ldb * 4), (uint32_t)a.ldb, n0, a.N);
    } else {
        bl.init(bbase, (uint32_t)(a.N * a.ldb * 4), (uint32_t)a.ldb, n0, a.N, k_end);
    }

    f32x16 acc[WT::TM][WT::TN];
    const int nslices = (k_end - k_begin + BK - 1) / BK;
    gemm_mainloop<BM, BN, BK, kStages>(al, bl, As, Bs, acc, k_begin, nslices, tid, lane, wm0, wn0, ZeroAcc{});

    // Epilogue: C values of a column block are loaded before any store.
    const int h = lane >> 5;
    const int l32 = lane & 31;
    constexpr int NR = WT::TM * 16;
#pragma unroll
    for (int j = 0; j < WT::TN; ++j) {
        const int n = n0 + wn0 + j * 32 + l32;
        if (n >= a.N) continue;
        if constexpr (SPLIT) {
#pragma unroll
            for (int q = 0; q < NR; ++q) {
                const int m = m0 + wm0 + (q >> 4) * 32 + 8 * ((q & 15) >> 2) + 4 * h + (q & 3);
                if (m < a.M) a.ws[((int64_t)z * a.M + m) * a.N + n] = acc[q >> 4][j][q & 15];
            }
        } else if (a.c_mode == 0 && m0 + BM <= a.M) {
            // no C and every row of the tile exists (the batched Winograd GEMMs):
            // no per-element test or C load
            float *yp = a.y + batch * a.stride_y + (int64_t)(m0 + wm0 + 4 * h) * a.N + n;
#pragma unroll
            for (int q = 0; q < NR; ++q)
                yp[(int64_t)((q >> 4) * 32 + 8 * ((q & 15) >> 2) + (q & 3)) * a.N] = a.alpha * acc[q >> 4][j][q & 15];
        } else {
            float cv[NR];
#pragma unroll
            for (int q = 0; q < NR; ++q) {
                const int m = m0 + wm0 + (q >> 4) * 32 + 8 * ((q & 15) >> 2) + 4 * h + (q & 3);
                float c = 0.f;
                if (m < a.M) {
                    if (a.c_mode == 1) c = a.c[n];
                    else if (a.c_mode == 2) c = a.c[(int64_t)m * a.N + n];
                }
                cv[q] = c;
            }
#pragma unroll
            for (int q = 0; q < NR; ++q) {
                const int m = m0 + wm0 + (q >> 4) * 32 + 8 * ((q & 15) >> 2) + 4 * h + (q & 3);
                if (m < a.M) a.y[batch * a.stride_y + (int64_t)m * a.N + n] = a.alpha * acc[q >> 4][j][q & 15] + a.beta * cv[q];
            }
        }
    }
}

__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float *__restrict__ ws, int nsplit, int M,
                                                                 int N, float alpha, float beta, int c_mode,
                                                                 const float *__restrict__ c,
                                                                 float *__restrict__ y) {
    const int64_t total = (int64_t)M * N;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        float v = splitk_sum(ws, nsplit, total, e);
        v *= alpha;
        if (c_mode == 1) v += beta * c[e % N];
        else if (c_mode == 2) v += beta * c[e];
        y[e] = v;
    }
}

// Y = alpha * A B^T (+ beta C) for at most MR rows, A [M][K] and B [N][K] both
// row-major with K contiguous (the Gemm transB=1 layout of fully-connected
// layers): KS waves per output column stream its row of B once, in float4s
// when K % 4 == 0 and both bases are 16-byte aligned, against the M rows of A
// (L2-resident), then sum each row's lane partials with a shuffle tree. The
// whole launch reads B once from HBM; the MFMA tiles would stage it through
// LDS for a single row of A. A workgroup serves 4 columns; with KS > 1 each
// wave of a column takes a contiguous 1/KS of K and the first of them adds the
// others' sums (through LDS, in part order), so more loads are in flight per
// column on the same number of workgroups (gemv_k_parts picks KS).
template <int MR, bool VEC, int KS>
__global__ __launch_bounds__(1024) void gemv_rows_kernel(const float *__restrict__ A, const float *__restrict__ B,
                                                        const float *__restrict__ Cm, int c_mode, float alpha,
                                                        float beta, float *__restrict__ Y, int M, int N, int K) {
    static_assert(KS == 1 || KS == 2 || KS == 4, "K parts per column: 1, 2 or 4");
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int n = blockIdx.x * 4 + w / KS;
    const int kp = w % KS;
    const bool live = n < N;
    if constexpr (KS == 1) {
        if (!live) return; // whole wave; no barrier follows
    }
    const float *bp = B + (int64_t)(live ? n : 0) * K;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    if (live) {
        if constexpr (VEC) {
            const int k4 = K >> 2;
            const int beg = (int)((int64_t)kp * k4 / KS), end = (int)((int64_t)(kp + 1) * k4 / KS);
#pragma unroll 4
            for (int j = beg + lane; j < end; j += 64) {
                const f32x4 b = *reinterpret_cast<const f32x4 *>(bp + 4 * j);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    if (m < M) {
                        const f32x4 av = *reinterpret_cast<const f32x4 *>(A + (int64_t)m * K + 4 * j);
                        acc[m] += av[0] * b[0] + av[1] * b[1] + av[2] * b[2] + av[3] * b[3];
                    }
                }
            }
        } else {
            const int beg = (int)((int64_t)kp * K / KS), end = (int)((int64_t)(kp + 1) * K / KS);
            for (int k = beg + lane; k < end; k += 64) {
                const float b = bp[k];
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    if (m < M) acc[m] += A[(int64_t)m * K + k] * b;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
    if constexpr (KS > 1) {
        __shared__ float red[4 * KS][MR];
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m) red[w][m] = acc[m];
        }
        __syncthreads();
        if (kp != 0 || !live) return;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float s = red[w][m];
#pragma unroll
            for (int p = 1; p < KS; ++p) s += red[w + p][m];
            acc[m] = s;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m >= M) break;
            float v = acc[m] * alpha;
            if (c_mode == 1) v += beta * Cm[n];
            else if (c_mode == 2) v += beta * Cm[(int64_t)m * N + n];
            Y[(int64_t)m * N + n] = v;
        }
    }
}

// Tag the loaders with their source orientation for gemm_kernel.
template <int BT, int BK, bool VEC>
struct KMajorG : KMajorLoader<BT, BK, VEC> {
    static constexpr bool kIsKMajor = true;
};
template <int BT, int BK, bool VEC>
struct RowKG : RowKLoader<BT, BK, VEC> {
    static constexpr bool kIsKMajor = false;
};

// ---- Gemm ----
namespace {

template <int BM, int BN, class AL, class BL>
int launch_gemm_tile(const GemmKArgs &a, int batch, int split, hipStream_t st) {
    dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, split > 1 ? split : batch);
    if (split > 1)
        hipLaunchKernelGGL((gemm_kernel<BM, BN, kBK, AL, BL, true>), grid, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, BN, kBK, AL, BL, false>), grid, dim3(kThreads), 0, st, a);
    return check_launch();
}

template <int BM, int BN, bool TA, bool TB, bool VA, bool VB>
int launch_gemm_cfg(const GemmKArgs &a, int batch, int split, hipStream_t st) {
    // A: trans_a -> source [K][M] (k-major); else [M][K] (rows, K contiguous).
    // B: trans_b -> source [N][K] (rows, K contiguous); else [K][N] (k-major).
    using AL = typename std::conditional<TA, KMajorG<BM, kBK, VA>, RowKG<BM, kBK, VA>>::type;
    using BL = typename std::conditional<TB, RowKG<BN, kBK, VB>, KMajorG<BN, kBK, VB>>::type;
    return launch_gemm_tile<BM, BN, AL, BL>(a, batch, split, st);
}

template <int BM, int BN, bool TA, bool TB, bool VA>
int gemm_pick_vb(const GemmKArgs &a, bool vb, int batch, int split, hipStream_t st) {
    return vb ? launch_gemm_cfg<BM, BN, TA, TB, VA, true>(a, batch, split, st)
              : launch_gemm_cfg<BM, BN, TA, TB, VA, false>(a, batch, split, st);
}

template <int BM, int BN, bool TA, bool TB>
int gemm_pick_va(const GemmKArgs &a, bool va, bool vb, int batch, int split, hipStream_t st) {
    return va ? gemm_pick_vb<BM, BN, TA, TB, true>(a, vb, batch, split, st)
              : gemm_pick_vb<BM, BN, TA, TB, false>(a, vb, batch, split, st);
}

template <int BM, int BN, bool TA>
int gemm_pick_tb(const GemmKArgs &a, bool tb, bool va, bool vb, int batch, int split, hipStream_t st) {
    return tb ? gemm_pick_va<BM, BN, TA, true>(a, va, vb, batch, split, st)
              : gemm_pick_va<BM, BN, TA, false>(a, va, vb, batch, split, st);
}

template <int BM, int BN>
int launch_gemm_loaders(const GemmKArgs &a, bool ta, bool tb, bool va, bool vb, int batch, int split,
                        hipStream_t st) {
    return ta ? gemm_pick_tb<BM, BN, true>(a, tb, va, vb, batch, split, st)
              : gemm_pick_tb<BM, BN, false>(a, tb, va, vb, batch, split, st);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

TileChoice gemm_tiles(const SpinnHipGemmDesc *d) {
    return choose_tiles(d->m, d->n, d->k, d->batch > 0 ? d->batch : 1, d->batch <= 1);
}

// The shapes gemm_run hands to gemv_rows_kernel (no workspace).
bool gemm_is_gemv(const SpinnHipGemmDesc *d) {
    return (d->batch <= 1) && d->m <= 4 && !d->trans_a && d->trans_b;
}

// Waves per output column in gemv_rows_kernel (graph-replayed on MI355X, weights
// MALL-resident / after a 512 MiB flush): 1000 x 2048 with one row of A 3.52 /
// 9.4 us on one wave per column, 3.38 / 8.2 on two, 3.77 / 7.5 on four; with
// four rows 6.3 / 18.8 on one, 5.0 / 10.6 on four. K = 600 (2.90 against 3.11
// us on two waves) and 4096 columns (12.9 against 13.3 us) keep one wave.
int gemv_k_parts(int M, int N, int K) {
    if (N >= 2048 || K < 1024) return 1;
    return M == 1 ? 2 : 4;
}

} // namespace

static int gemm_wavek(const SpinnHipGemmDesc *d) {
    return wavek_tile(d->m, d->n, d->k, d->batch > 0 ? d->batch : 1, kWkGemm);
}

size_t gemm_workspace_bytes(const SpinnHipGemmDesc *d) {
    if (gemm_is_gemv(d) || gemm_wavek(d)) return 0;
    TileChoice tc = gemm_tiles(d);
    if (tc.split <= 1) return 0;
    return (size_t)tc.split * d->m * (size_t)d->n * sizeof(float);
}

int gemm_run(const SpinnHipGemmDesc *d, const float *A, const float *B, const float *C, float *Y, void *ws,
             size_t ws_bytes, hipStream_t st) {
    GemmKArgs a{};
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
    // Buffer descriptors address at most 2 GiB per operand.
    const uint64_t a_bytes = (uint64_t)d->m * d->k * sizeof(float);
    const uint64_t b_bytes = (uint64_t)d->n * d->k * sizeof(float);
    if (a_bytes > kMaxOperandBytes || b_bytes > kMaxOperandBytes) return SPINN_HIP_EUNSUPPORTED;
    // Vector loads need 16-byte aligned rows in every batch entry.
    const bool va = aligned16(A) && (a.lda % 4 == 0) && (batch == 1 || d->stride_a % 4 == 0);
    const bool vb = aligned16(B) && (a.ldb % 4 == 0) && (batch == 1 || d->stride_b % 4 == 0);
    if (gemm_is_gemv(d)) {
        // fully-connected shape: B streamed once by waves, no tiles, no workspace
        const int ks = gemv_k_parts(d->m, d->n, d->k);
        const dim3 grid((unsigned)((d->n + 3) / 4));
        const bool vec = va && vb;
#define SPINN_GEMV(VEC, KS)                                                                                      \
    hipLaunchKernelGGL((gemv_rows_kernel<4, VEC, KS>), grid, dim3(256 * KS), 0, st, A, B, C, a.c_mode, d->alpha,   \
                       d->beta, Y, d->m, d->n, d->k)
        if (ks == 4) {
            if (vec) SPINN_GEMV(true, 4);
            else SPINN_GEMV(false, 4);
        } else if (ks == 2) {
            if (vec) SPINN_GEMV(true, 2);
            else SPINN_GEMV(false, 2);
        } else {
            if (vec) SPINN_GEMV(true, 1);
            else SPINN_GEMV(false, 1);
        }
#undef SPINN_GEMV
        return check_launch();
    }
    if (const int ts = gemm_wavek(d)) return wavek_gemm(d, ts, A, B, C, Y, st);
    TileChoice tc = gemm_tiles(d);
    if (tc.split > 1) {
        const size_t need = (size_t)tc.split * d->m * (size_t)d->n * sizeof(float);
        if (!ws || ws_bytes < need) return SPINN_HIP_EWORKSPACE;
        a.ws = (float *)ws;
        a.k_chunk = tc.k_chunk;
    }
    const bool ta = d->trans_a != 0, tb = d->trans_b != 0;
    int rc;
    if (tc.bm == 128 && tc.bn == 128) rc = launch_gemm_loaders<128, 128>(a, ta, tb, va, vb, batch, tc.split, st);
    else if (tc.bm == 128 && tc.bn == 64) rc = launch_gemm_loaders<128, 64>(a, ta, tb, va, vb, batch, tc.split, st);
    else if (tc.bm == 64 && tc.bn == 128) rc = launch_gemm_loaders<64, 128>(a, ta, tb, va, vb, batch, tc.split, st);
    else if (tc.bm == 32 && tc.bn == 128) rc = launch_gemm_loaders<32, 128>(a, ta, tb, va, vb, batch, tc.split, st);
    else rc = launch_gemm_loaders<64, 64>(a, ta, tb, va, vb, batch, tc.split, st);
    if (rc) return rc;
    if (tc.split > 1) {
        const int64_t total = (int64_t)d->m * d->n;
        const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
        hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, (const float *)ws, tc.split,
                           d->m, d->n, d->alpha, d->beta, a.c_mode, C, Y);
        rc = check_launch();
    }
    return rc;
}

} // namespace spinn
