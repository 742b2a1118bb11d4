/*
 * spinn_hip.h - C ABI of the HIP (gfx950) compute layer.
 *
 * Plain C: plain pointers, sizes and small descriptor structs, no HIP or torch
 * types (a hipStream_t is passed as void*, NULL = the null stream). Every
 * pointer argument of a compute entry point is a DEVICE address. Entry points
 * return 0 on success or a negative SPINN_HIP_E* code; they never allocate
 * device memory: scratch comes in through `workspace`, sized by the matching
 * *_workspace_size() query, and pre-laid-out weights through `packed_w`.
 *
 * Which reference interface each entry point replaces is noted on it.
 */
#ifndef SPINN_AMD_HIP_H
#define SPINN_AMD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPINN_HIP_OK 0
#define SPINN_HIP_EINVAL (-1)      /* bad arity / shape / argument (reference ops return -1) */
#define SPINN_HIP_EUNSUPPORTED (-2) /* valid request this layer does not implement */
#define SPINN_HIP_EWORKSPACE (-3)   /* workspace missing or too small */
#define SPINN_HIP_EDEVICE (-4)      /* a kernel reported an internal failure (spinn_hip_device_status) */
#define SPINN_HIP_ERUNTIME (-100)   /* HIP runtime error: code = -100 - hipError_t */

/* Convolution algorithms. AUTO picks per shape (see spinn_hip_conv_select_algo). */
enum {
    SPINN_CONV_ALGO_AUTO = 0,
    SPINN_CONV_ALGO_IMPLICIT_GEMM = 1, /* im2col fused into the tile load; 1x1 s1 p0 reads X directly */
    SPINN_CONV_ALGO_WINOGRAD = 2,      /* F(2x2,3x3), 3x3 s1 group 1 only; needs packed_w */
    SPINN_CONV_ALGO_DIRECT = 3,        /* grouped / depthwise direct convolution */
    SPINN_CONV_ALGO_WINOGRAD_F43 = 4   /* F(4x4,3x3), same eligibility and operands as WINOGRAD */
};

/*
 * Conv2d + fused epilogue, NCHW fp32.
 *   y[n,oc,oh,ow] = post( sum_{c,kh,kw} w[oc,c,kh,kw] * x[n, g*C/g + c, oh*sh-ph+kh, ow*sw-pw+kw] )
 *   post(v): v += bias[oc] (if bias); if act in {ADD, ADD_RELU}: v += residual[n,oc,oh,ow];
 *            if act in {RELU, ADD_RELU}: v = max(v,0); else if act == SILU: v = v/(1+exp(-v)).
 * Only the begin pads are used and dilations are ignored, as in
 * SPINN/run_time/ops/conv/conv2d.c:124-142; the epilogue order is
 * SPINN/run_time/ops/mm/gemm_kernel.c:316-338 with the codes of SPINN/graph_opt.h:31-36.
 */
typedef struct {
    int32_t n, c, h, w;     /* input */
    int32_t oc, oh, ow;     /* output */
    int32_t kh, kw;         /* kernel */
    int32_t sh, sw;         /* strides */
    int32_t ph, pw;         /* begin pads */
    int32_t group;          /* C and OC divisible by group */
    int32_t act;            /* SPINN_ACT_* */
    int32_t algo;           /* SPINN_CONV_ALGO_* */
    int32_t reserved;
} SpinnHipConvDesc;

/* Replaces the arithmetic of op_conv2d (SPINN/run_time/ops/conv/conv2d.c:92-232):
 * im2col (:14-79) + sgemm_nn_packed_a / sgemm_nn (SPINN/run_time/ops/mm/gemm_kernel.c:304-339,497-590),
 * the Winograd path (SPINN/run_time/ops/conv/winograd.c:96-210) and the grouped loop (:178-227).
 * bias may be NULL; residual must be non-NULL iff act is ADD or ADD_RELU. */
int spinn_hip_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed_w,
                   const float *bias, const float *residual, float *y, void *workspace,
                   size_t workspace_bytes, void *stream);

/*
 * spinn_hip_conv without a workspace argument: its scratch (split-K partial
 * sums, Winograd V and M) is a fixed device array of
 * SPINN_HIP_NOALLOC_SCRATCH_BYTES held by the library. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc), and
 * once spinn_hip_init has run for its device it calls no allocating routine.
 * The caller still passes inputs (including
 * packed_w from spinn_hip_conv_pack_weights) and the output; results are those
 * of spinn_hip_conv. A descriptor whose spinn_hip_conv_workspace_size exceeds
 * the array returns SPINN_HIP_EWORKSPACE without launching. Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other host threads) race. Nothing in the array needs to start at zero.
 * spinn_hip_init resolves the array's device address and runs the
 * once-per-device XCD placement check the stream-K plan reads (a 16 KB
 * allocation, freed); without it the first call on a device does both.
 */
#define SPINN_HIP_NOALLOC_SCRATCH_BYTES (128u << 20) /* every conv of ResNet-101 b32, VGG b8, YOLOv10n b16 */
int spinn_hip_conv_noalloc(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed_w,
                           const float *bias, const float *residual, float *y, void *stream);

/* Algorithm AUTO would run for this shape (never returns AUTO). */
int spinn_hip_conv_select_algo(const SpinnHipConvDesc *d);
/* Device scratch bytes spinn_hip_conv needs for this descriptor (0 = none). */
size_t spinn_hip_conv_workspace_size(const SpinnHipConvDesc *d);
/* Bytes of pre-laid-out weights the selected algorithm needs (0 = reads w directly).
 * Replaces sgemm_pack_a_offline / winograd_pack_weight
 * (SPINN/run_time/ops/mm/gemm_kernel.c:346-369, SPINN/run_time/ops/conv/winograd.c:82-94). */
size_t spinn_hip_conv_packed_size(const SpinnHipConvDesc *d);
/* Fill `packed` (spinn_hip_conv_packed_size bytes) from w [OC, C/g, KH, KW]. */
int spinn_hip_conv_pack_weights(const SpinnHipConvDesc *d, const float *w, float *packed, void *stream);

/*
 * Gemm / MatMul, fp32 row-major.
 *   y[b] = alpha * op(A[b]) * op(B[b]) + beta * C    (op = transpose when trans_*)
 * A[b] is M x K (K x M when trans_a), B[b] is K x N (N x K when trans_b).
 * c_mode: 0 = no C, 1 = C is a vector [N] broadcast over rows, 2 = C is [M, N].
 * batch > 1 steps A, B and Y by stride_a / stride_b / stride_y elements
 * (stride_b = 0 broadcasts one B over the batch). C is never batched.
 * alpha scales only the product (the reference also scales the C prefill when
 * M > 1, SPINN/run_time/ops/mm/gemm_kernel.c:298-301; parity is held to the
 * operator's definition, which the reference configs hit with alpha = 1).
 */
typedef struct {
    int32_t m, n, k;
    int32_t trans_a, trans_b;
    int32_t c_mode;
    float alpha, beta;
    int32_t batch;
    int32_t reserved;
    int64_t stride_a, stride_b, stride_y;
} SpinnHipGemmDesc;

/* Replaces op_gemm (SPINN/run_time/ops/mm/gemm.c:7-78) and op_matmul
 * (SPINN/run_time/ops/mm/matmul.c:6-62) over sgemm_tiled (gemm_kernel.c:206-302). */
int spinn_hip_gemm(const SpinnHipGemmDesc *d, const float *a, const float *b, const float *c, float *y,
                   void *workspace, size_t workspace_bytes, void *stream);
size_t spinn_hip_gemm_workspace_size(const SpinnHipGemmDesc *d);

/* ---- glue operators around the conv/GEMM path ---- */

typedef struct {
    int32_t n, c, h, w;
    int32_t oh, ow;
    int32_t kh, kw, sh, sw, ph, pw;
} SpinnHipPoolDesc;

/* MaxPool2d; a window with no valid tap yields -1e30 (SPINN/run_time/ops/pool/maxpool.c:5-49). */
int spinn_hip_maxpool2d(const SpinnHipPoolDesc *d, const float *x, float *y, void *stream);

/* Mean over the middle axis of an [outer, dim, inner] view
 * (SPINN/run_time/ops/reduce/reduce_mean.c:62-75; GlobalAveragePool is outer=N*C, dim=H*W, inner=1,
 * SPINN/run_time/ops/pool/global_avg_pool.c:4-28). */
int spinn_hip_reduce_mean(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y,
                          void *stream);

/* Device-to-device copy (regions must not overlap) for Reshape / Flatten / Identity
 * (SPINN/run_time/ops/shape/reshape.c:6-14, SPINN/run_time/ops/tensor/flatten.c:3-8). */
int spinn_hip_copy(void *dst, const void *src, size_t bytes, void *stream);

/* ---- unfused graph nodes: elementwise, normalisation, layout (fp32) ---- */

enum { SPINN_BINARY_ADD = 0, SPINN_BINARY_SUB = 1, SPINN_BINARY_MUL = 2, SPINN_BINARY_DIV = 3 };

/* y[i] = a[i % na] (op) b[i % nb] for 0 <= i < n: the reference's broadcast rule
 * (SPINN/run_time/ops/math/add.c:14-19, sub.c:16-18, mul.c:20-60). DIV replaces
 * a divisor with |b| < 1e-6 by +1e-6 (SPINN/run_time/ops/math/div.c:24-28).
 * n, na, nb < 2^32 (the reference's element counts are uint32). */
int spinn_hip_binary(int op, const float *a, int64_t na, const float *b, int64_t nb, float *y, int64_t n,
                     void *stream);

enum { SPINN_UNARY_RELU = 0, SPINN_UNARY_SIGMOID = 1, SPINN_UNARY_SILU = 2 };

/* y = max(x, 0) (SPINN/run_time/ops/activation/relu.c:4-16), y = 1/(1+exp(-x))
 * (SPINN/run_time/ops/activation/sigmoid.c:7-25), y = x/(1+exp(-x)). */
int spinn_hip_unary(int op, const float *x, float *y, int64_t n, void *stream);

/* Inference BatchNormalization over x [n, c, spatial]:
 * alpha = scale[c] / sqrt(var[c] + eps), y = x * alpha + (bias[c] - mean[c] * alpha)
 * (SPINN/run_time/ops/norm/batch_norm.c:17-76). */
int spinn_hip_batchnorm(int64_t n, int64_t c, int64_t spatial, const float *x, const float *scale,
                        const float *bias, const float *mean, const float *var, float eps, float *y,
                        void *stream);

/* Softmax over the middle axis of an [outer, dim, inner] view: y = exp(x - max) / sum
 * (SPINN/run_time/ops/activation/softmax.c:109-170). */
int spinn_hip_softmax(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, void *stream);

/* One strided block copy of a Concat input or a Split output: for o < outer and
 * j < len, dst[o * dst_row + dst_off + j] = src[o * src_row + src_off + j] (elements). */
typedef struct {
    const float *src;
    float *dst;
    int64_t src_row, src_off;
    int64_t dst_row, dst_off;
    int64_t len;
} SpinnHipBlockCopy;

#define SPINN_HIP_MAX_BLOCKS 16

/* Concat (SPINN/run_time/ops/tensor/concat.c:5-26) and Split
 * (SPINN/run_time/ops/tensor/split.c:5-26) as up to SPINN_HIP_MAX_BLOCKS block
 * copies in one launch; blocks must not overlap in dst. */
int spinn_hip_block_copy(const SpinnHipBlockCopy *blocks, int n_blocks, int64_t outer, void *stream);

/* Transpose of an ndim <= 8 tensor of < 2^32 elements: y's dim d is x's dim perm[d]
 * (SPINN/run_time/ops/shape/transpose.c:14-104; perm = NULL reverses the dims, as there). */
int spinn_hip_transpose(int ndim, const int64_t *dims, const int32_t *perm, const float *x, float *y,
                        void *stream);

/* Nearest Resize of nc planes h x w -> oh x ow: y[p, i, j] = x[p, i*h/oh, j*w/ow]
 * with integer division (SPINN/run_time/ops/tensor/resize.c:4-31). */
int spinn_hip_resize_nearest(int64_t nc, int32_t h, int32_t w, int32_t oh, int32_t ow, const float *x, float *y,
                             void *stream);

/* ---- detector post-processing: ReduceMax, TopK, GatherElements, Tile, Cast, integer Div/Mod ---- */

/* y[i] = max over x[i * block .. i * block + block) for i < rows, taken in index
 * order from the first element with `>` (SPINN/run_time/ops/reduce/reduce_max.c:4-28:
 * block = |x| / |y|). Rows containing NaN are outside the parity contract. */
int spinn_hip_reduce_max(int64_t rows, int64_t block, const float *x, float *y, void *stream);

/* TopK over the last axis of rows x n (SPINN/run_time/ops/tensor/topk.c:20-89): the k
 * largest values of each row, sorted descending, ties in ascending index order (the
 * reference sorts (value, index) pairs with glibc qsort, a stable merge sort, under
 * `a > b`; -0.0 and +0.0 compare equal). values [rows, k] fp32, indices [rows, k] int64.
 * 1 <= k <= min(n, SPINN_HIP_TOPK_MAX_K). NaN inputs are outside the parity contract. */
#define SPINN_HIP_TOPK_MAX_K 1024
int spinn_hip_topk(int64_t rows, int64_t n, int64_t k, const float *x, float *values, int64_t *indices,
                   void *stream);

/* GatherElements (SPINN/run_time/ops/tensor/gather_elements.c:5-76): for every output
 * coordinate c, y[c] = data[c with c[axis] replaced by idx[c]]; idx < 0 wraps once by
 * in_dims[axis], an index still outside [0, in_dims[axis]) reads position 0, as in the
 * reference. index_dtype is ENNF_TYPE_INT64 (7) or ENNF_TYPE_INT32 (6). */
typedef struct {
    int32_t ndim;        /* 1..8 */
    int32_t axis;        /* normalised, 0 <= axis < ndim */
    int32_t index_dtype; /* 6 = int32, 7 = int64 */
    int32_t reserved;
    int64_t in_dims[8];  /* data */
    int64_t out_dims[8]; /* indices and y */
} SpinnHipGatherDesc;
int spinn_hip_gather_elements(const SpinnHipGatherDesc *d, const float *data, const void *indices, float *y,
                              void *stream);

/* Tile (SPINN/run_time/ops/tensor/tile.c:6-65): y[c] = x[c mod in_dims] per axis for
 * every output coordinate c; elements of elem_bytes in {1, 2, 4, 8}. */
int spinn_hip_tile(int ndim, const int64_t *in_dims, const int64_t *out_dims, int elem_bytes, const void *x,
                   void *y, void *stream);

/* Cast between ENNF_TYPE_FLOAT32 / INT32 / INT64 (SPINN/run_time/ops/tensor/cast.c:13-73):
 * int -> float rounds to nearest, float -> int truncates toward zero, int64 -> int32
 * keeps the low 32 bits; equal types copy. Other pairs: SPINN_HIP_EUNSUPPORTED. */
int spinn_hip_cast(int src_dtype, int dst_dtype, int64_t n, const void *x, void *y, void *stream);

/* Integer / remainder forms of Div and Mod with the modulo broadcast of
 * spinn_hip_binary, y[i] = a[i % na] (op) b[i % nb]:
 *   SPINN_BINARY_DIV on int32 / int64: C division truncating toward zero, 0 where b == 0
 *     (SPINN/run_time/ops/math/div.c:33-48);
 *   SPINN_BINARY_MOD on int32 / int64: C remainder (sign of a), 0 where b == 0;
 *     on fp32: fmodf (SPINN/run_time/ops/math/mod.c:18-45). */
enum { SPINN_BINARY_MOD = 4 };
int spinn_hip_binary_typed(int op, int dtype, const void *a, int64_t na, const void *b, int64_t nb, void *y,
                           int64_t n, void *stream);

/* ---- device, memory, stream, event and graph plumbing for the host runtime ---- */

int spinn_hip_init(int device);
int spinn_hip_device_count(int *count);
int spinn_hip_malloc(void **ptr, size_t bytes);
int spinn_hip_free(void *ptr);
int spinn_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int spinn_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
/* Fill `bytes` (multiple of 4) with a 32-bit pattern using a kernel (graph-safe, no memset node). */
int spinn_hip_fill_u32(void *dst, uint32_t value, size_t bytes, void *stream);
int spinn_hip_stream_create(void **stream);
int spinn_hip_stream_destroy(void *stream);
int spinn_hip_stream_sync(void *stream);
int spinn_hip_event_create(void **event);
int spinn_hip_event_destroy(void *event);
int spinn_hip_event_record(void *event, void *stream);
int spinn_hip_event_elapsed_ms(void *start, void *stop, float *ms);
int spinn_hip_graph_capture_begin(void *stream);
int spinn_hip_graph_capture_end(void *stream, void **graph_exec);
int spinn_hip_graph_launch(void *graph_exec, void *stream);
int spinn_hip_graph_destroy(void *graph_exec);
const char *spinn_hip_error_string(int code);

/* Tuning hook: force the MFMA GEMM output tile (bm, bn in {64, 128}) and K
 * split for every later conv/Gemm launch and workspace query; bm = bn = 32
 * (or 16) forces the wave-K kernel (32 x 32 or 16 x 16 tiles, K split over a
 * workgroup's waves);
 * bm = 0 restores the per-shape choice. Change it only between plans: packed weights do not
 * depend on it, workspace sizes do. No counterpart in the reference. */
void spinn_hip_tune_force_tiles(int bm, int bn, int split);

/* Tuning hook: the data-parallel + stream-K split of the implicit-GEMM conv
 * (whole tiles one workgroup each, the tiles left over after an even share
 * per CU cut along K and finished in the same launch): -1 = per-shape choice
 * (default, or SPINN_STREAMK=0|1 from the environment), 0 = never, 1 = for
 * every grid of at least one tile per CU whose tile count is not a multiple
 * of the CU count, 2 = as 1 with the parts' sums exchanged through memory
 * even where spinn_hip_init found them sharing an L2. Change it only between
 * plans: workspace sizes depend on it. No counterpart in the reference. */
void spinn_hip_tune_streamk(int mode);

/* Tuning hook: how F(4x4,3x3) Winograd layers run. -1 = per-shape choice (default,
 * or SPINN_WINOGRAD_FUSED=0|1 from the environment), 0 = always three launches
 * (input transform, 36 batched GEMMs, output transform, V and M in the workspace),
 * 1 = one fused launch wherever it fits (transforms and GEMMs on chip, no workspace).
 * Change it only between plans: workspace sizes depend on it. No counterpart in the
 * reference. */
void spinn_hip_tune_winograd_fused(int mode);

/* Test hook: arrival rounds of the stream-K parts (default 4; < 0 restores
 * it). 0 makes every arrival fail, so the cut tiles stay unwritten and the
 * status word reports it, while every kernel still exits normally. No
 * counterpart in the reference. */
void spinn_hip_tune_streamk_tries(int tries);

/* Device-side failure report: SPINN_HIP_EDEVICE when a kernel launched since
 * the last call could not finish its work (a stream-K tile whose parts' arrival
 * protocol broke, leaving the tile unwritten), else 0; clears the report. Call
 * after synchronising the streams the launches ran on; spinn_run does. The
 * word is host memory the kernels write, allocated by spinn_hip_init or the
 * first workspace query of a stream-K conv. No counterpart in the reference
 * (its operators run on the calling thread and return their errors). */
int spinn_hip_device_status(void);

/* Library version / build identification string. */
const char *spinn_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif /* SPINN_AMD_HIP_H */
