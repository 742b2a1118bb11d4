// spinn_hip_internal.h - declarations shared by the HIP translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <algorithm>
#include <stdint.h>
#include "../../include/spinn_hip.h"
#include "../../include/ennf_format.h"

namespace spinn {

// Map the last launch error to the C-ABI code (0 when the launch was accepted).
inline int hip_code(hipError_t e) { return e == hipSuccess ? 0 : (SPINN_HIP_ERUNTIME - (int)e); }
inline int check_launch() { return hip_code(hipGetLastError()); }

// SiLU v / (1 + e^-v) as v * rcp(1 + 2^(-v log2 e)) through the hardware exp2
// and reciprocal (about 1 ulp each): 5 instructions against about 20 for a
// correctly rounded expf and division, a relative difference of a few 1e-7
// (the log2 e product's rounding grows it with |v|: 1e-6 at |v| = 16). Large
// negative v give -0 (e^-v overflows to inf, its reciprocal to 0).
__device__ __forceinline__ float silu(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}

// Fused post-op after bias and residual (SPINN/run_time/ops/mm/gemm_kernel.c:324-335).
__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == SPINN_ACT_RELU || act == SPINN_ACT_ADD_RELU) {
        v = v < 0.f ? 0.f : v;
    } else if (act == SPINN_ACT_SILU) {
        v = silu(v);
    }
    return v;
}

// The fused post-op as a compile-time class: 0 = none (NONE, CLIP, ADD), 1 = ReLU
// (RELU, ADD_RELU), 3 = SiLU; the bias and residual are added before it.
__host__ __device__ constexpr int act_class(int act) {
    return (act == SPINN_ACT_RELU || act == SPINN_ACT_ADD_RELU) ? 1 : (act == SPINN_ACT_SILU ? 3 : 0);
}
template <int AC>
__device__ __forceinline__ float apply_act_c(float v) {
    if constexpr (AC == 1) return v < 0.f ? 0.f : v;
    else if constexpr (AC == 3) return silu(v);
    else return v;
}

// Sum of the split-K partials ws[s * plane + e] for s = 0..nsplit-1, added in
// split order starting from 0 (the order the partials' K ranges take). The
// loads of a group of 8 splits (all of them, up to 16) are issued before the
// first add: a plain loop would wait out one memory round trip per split.
__device__ __forceinline__ float splitk_sum(const float *__restrict__ ws, int nsplit, int64_t plane, int64_t e) {
    float v = 0.f;
    if (nsplit > 8 && nsplit <= 16) {
        // 9..16 splits (the tile rule's largest): every split's load in flight at
        // once, one memory round trip instead of two; the same split-order sum
        float p[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) p[u] = ws[(int64_t)min(u, nsplit - 1) * plane + e];
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (u < nsplit) v += p[u];
        return v;
    }
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
        float p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p[u] = ws[(int64_t)min(s0 + u, nsplit - 1) * plane + e];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (s0 + u < nsplit) v += p[u];
    }
    return v;
}

constexpr int kBK = 16;    // K depth of one LDS slice of the MFMA GEMMs
// Register stages of the K loop (global loads run that many slices ahead of
// their LDS write). Measured on the ResNet-101 batch-32 and batch-1 conv
// shapes: 4 stages were no faster than 2 (the loads are not the stall), and
// cost registers, so 2.
constexpr int kStages = 2;

// Output tile (bm x bn) and K split of one MFMA GEMM launch.
struct TileChoice {
    int bm, bn, split, k_chunk;
};
TileChoice choose_tiles(int M, int N, int K, int reps, bool allow_split);
void force_tiles(int bm, int bn, int split);
// Data-parallel + stream-K split of one launch (streamk.h): dp_per_xcd whole
// tiles per XCD, the R remaining tiles cut along K, either over W extra
// workgroups per XCD (scheme kSkSplitWgs) or in p parts done by whole-tile
// workgroups (kSkPartsInDp). Workspace: cnt_bytes of arrival counters, then
// the partial-tile slots.
struct SkPlan {
    int dp_per_xcd, R, scheme, W, p, grid;
    size_t cnt_bytes, ws_bytes;
};
// False when whole tiles are balanced enough (or the split is switched off).
bool plan_streamk(int tiles_m, int tiles_n, int S, int tile_elems, SkPlan &p);
void force_streamk(int mode);
uint64_t streamk_epoch();
// Host-visible status word that kernels set when an internal protocol fails
// (a stream-K arrival that cannot complete): allocated once per process at
// set-up (spinn_hip_init, or the plan-time workspace query); null before.
void init_device_status();
unsigned *device_status_word();
// Read and clear the word (the caller has synchronised the streams).
int take_device_status();
// Arrival rounds of the stream-K parts (4; a test hook sets 0 to force the
// failure report with every kernel still exiting normally).
void force_streamk_tries(int tries);
int streamk_tries();
// Check once per device that workgroup b runs on XCD b % 8 (so the parts of a
// cut tile can exchange sums through one L2); xcd_local_parts() reports the
// result for the current device, false until checked.
void probe_xcd_local(int device);
bool xcd_local_parts();
// Output tile edge of the wave-K kernel (K split over a workgroup's waves) for
// an (M x N x K) problem repeated `reps` times: 32 or 16, or 0 when it runs on the
// 64/128-wide tiles of choose_tiles. `kind`: what the operands are.
enum WkKind { kWkGemm, kWkConvGather, kWkConvPointwise }; // pointwise: 1x1 stride-1 unpadded conv
int wavek_tile(int M, int N, int K, int reps, WkKind kind);
// true while spinn_hip_tune_force_tiles holds a tile shape or a K split
bool tiles_forced();

// 7x7 stride-2 stems (stem_mfma.hip): C <= 4, OC <= 64, output rows <= 128 pixels,
// one workgroup per output row over an LDS-staged window; packed W^T as igemm_pack.
bool stem_mfma_eligible(const SpinnHipConvDesc *d);
int stem_mfma_conv(const SpinnHipConvDesc *d, const float *x, const float *packed, const float *bias,
                   const float *res, float *y, hipStream_t st);
// 3x3 stride-2 stems (stem_mfma.hip): C <= 4, OC <= 16, output rows <= 320 pixels, begin
// pads <= 1, one workgroup per output row on 16x16x4 MFMAs; raw weights W [OC][C][3][3].
bool stem3_mfma_eligible(const SpinnHipConvDesc *d);
int stem3_mfma_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias, const float *res,
                    float *y, hipStream_t st);

// wave-K kernels (wavek.hip): no workspace, packed conv weights as igemm_pack
int wavek_conv(const SpinnHipConvDesc *d, int ts, const float *x, const float *w, const float *packed, const float *bias,
               const float *res, float *y, hipStream_t st);
int wavek_gemm(const SpinnHipGemmDesc *d, int ts, const float *A, const float *B, const float *C, float *Y,
               hipStream_t st);

// Compute units of the current device (cached per device; 256 on MI355X).
int device_cu_count();

// Device address of spinn_hip_conv_noalloc's scratch array on `device` (the
// current device), resolved once per device (noalloc.hip).
int noalloc_scratch(int device, void **ptr);

// implicit GEMM (conv_gemm.hip)
int64_t igemm_packed_floats(const SpinnHipConvDesc *d);
// The k-contiguous tap-ordered weights [group][OCg][K] inside `packed`, or null
// when the layer's packing has none (1x1 windows, (c, kh, kw) order).
const float *igemm_kcopy(const SpinnHipConvDesc *d, const float *packed);
int igemm_pack(const SpinnHipConvDesc *d, const float *w, float *packed, hipStream_t st);
size_t igemm_workspace_bytes(const SpinnHipConvDesc *d);
int igemm_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed, const float *bias,
               const float *res, float *y, void *ws, size_t ws_bytes, hipStream_t st);
size_t gemm_workspace_bytes(const SpinnHipGemmDesc *d);
int gemm_run(const SpinnHipGemmDesc *d, const float *A, const float *B, const float *C, float *Y, void *ws,
             size_t ws_bytes, hipStream_t st);

// Winograd F(2x2,3x3) / F(4x4,3x3) (winograd.hip); m = output tile edge, 2 or 4
bool winograd_eligible(const SpinnHipConvDesc *d);
// F(4x4,3x3) in one launch (winograd_fused.hip): transforms and the 36 GEMMs on chip,
// no workspace; chosen per shape (few input channels) unless forced.
bool wino4_fused_selected(const SpinnHipConvDesc *d);
int wino4_fused_conv(const SpinnHipConvDesc *d, const float *x, const float *U, const float *bias,
                     const float *res, float *y, hipStream_t st);
void force_winograd_fused(int mode);
int64_t winograd_packed_floats(const SpinnHipConvDesc *d, int m);
int winograd_pack(const SpinnHipConvDesc *d, int m, const float *w, float *packed, hipStream_t st);
size_t winograd_workspace_bytes(const SpinnHipConvDesc *d, int m);
int winograd_conv(const SpinnHipConvDesc *d, int m, const float *x, const float *packed, const float *bias,
                  const float *res, float *y, void *ws, size_t ws_bytes, hipStream_t st);

// grouped / depthwise direct convolution (direct_conv.hip)
int direct_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *bias, const float *res,
                float *y, hipStream_t st);
// group 1, <= 4 input channels, 3x3 or 7x7: the stem kernel of direct_conv;
// stem_conv_pays: the shapes where AUTO prefers it
bool stem_conv_eligible(const SpinnHipConvDesc *d);
bool stem_conv_pays(const SpinnHipConvDesc *d);

// glue (glue.hip)
int maxpool2d(const SpinnHipPoolDesc *d, const float *x, float *y, hipStream_t st);
int reduce_mean(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, hipStream_t st);
int fill_u32(void *dst, uint32_t value, size_t bytes, hipStream_t st);

// unfused graph nodes (tensor_ops.hip)
int binary_op(int op, const float *a, int64_t na, const float *b, int64_t nb, float *y, int64_t n, hipStream_t st);
int unary_op(int op, const float *x, float *y, int64_t n, hipStream_t st);
int batchnorm(int64_t n, int64_t c, int64_t spatial, const float *x, const float *scale, const float *bias,
              const float *mean, const float *var, float eps, float *y, hipStream_t st);
int softmax(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, hipStream_t st);
int block_copy(const SpinnHipBlockCopy *blocks, int n_blocks, int64_t outer, hipStream_t st);
int transpose(int ndim, const int64_t *dims, const int32_t *perm, const float *x, float *y, hipStream_t st);
int resize_nearest(int64_t nc, int h, int w, int oh, int ow, const float *x, float *y, hipStream_t st);

// detector post-processing (postproc.hip)
int reduce_max_rows(int64_t rows, int64_t block, const float *x, float *y, hipStream_t st);
int topk_rows(int64_t rows, int64_t n, int k, const float *x, float *values, int64_t *indices, hipStream_t st);
int gather_elements(const SpinnHipGatherDesc *d, const float *data, const void *indices, float *y, hipStream_t st);
int tile(int ndim, const int64_t *in_dims, const int64_t *out_dims, int elem_bytes, const void *x, void *y,
         hipStream_t st);
int cast(int src, int dst, int64_t n, const void *x, void *y, hipStream_t st);
int binary_typed(int op, int dtype, const void *a, int64_t na, const void *b, int64_t nb, void *y, int64_t n,
                 hipStream_t st);

} // namespace spinn
