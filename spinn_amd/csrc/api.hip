// api.hip - the extern "C" entry points of include/spinn_hip.h: argument
// validation, algorithm selection, and the device/stream/graph plumbing the
// host runtime uses. All compute goes to the kernels in the other units.
#include "spinn_hip_internal.h"
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace spinn {

int device_cu_count() {
    static int cached[64];
    static std::once_flag once[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::call_once(once[dev], [dev]() {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cached[dev] = v;
    });
    return cached[dev];
}

static int env_winograd() {
    // SPINN_WINOGRAD=1 sends eligible 3x3 stride-1 convs to Winograd under AUTO,
    // 0 keeps them on the implicit GEMM; unset = per-shape choice.
    static int v = [] {
        const char *e = std::getenv("SPINN_WINOGRAD");
        if (!e || !*e) return -1;
        return e[0] == '0' ? 0 : 1;
    }();
    return v;
}

static int env_winograd_tile() {
    // SPINN_WINOGRAD_TILE=2|4 fixes the Winograd tile under AUTO; unset = per-shape choice.
    static int v = [] {
        const char *e = std::getenv("SPINN_WINOGRAD_TILE");
        if (!e || !*e) return 0;
        return e[0] == '2' ? 2 : 4;
    }();
    return v;
}

// AUTO's Winograd tile for an eligible 3x3 stride-1 conv: 4 (F(4,3)), 2 (F(2,3)) or
// 0 (stay on the implicit GEMM). Winograd cuts the GEMM flops 4x (F(4,3)) or 2.25x
// (F(2,3)) but moves V and M through memory in three launches, and its packed
// weights are 4x (F(4,3)) or 1.8x (F(2,3)) the raw ones. At small batch a layer's
// time is mostly its weight read, and a model's weights together compete for the
// 256 MB Infinity Cache: 22 ResNet-101 layers at 256@14x14 hold 207 MB as F(4,3)
// against 52 MB raw, which slows the 1x1 layers beside them too. Thresholds from
// whole-model graph replays and per-node times on MI355X (ResNet-101 at batch 1-32,
// YOLOv10n at 1, 4 and 16), with per-layer timings (weights cycled through copies
// larger than the cache) between them:
//  * 128+ channels in and out: at K >= 512 F(2,3) from 16 4x4 tiles (512@7x7
//    batch 8: 22.0 against 32.5 us for the implicit GEMM, the model step 17 us
//    faster) and F(4,3) from 48; at K = 256 F(4,3) from 64 tiles (256@14x14 batch 4:
//    21.1 against 23.9 us per node in the model; at 32 tiles, batch 2, 18.0 against
//    16.9); at K = 128 F(4,3) from 128 tiles.
//  * 64+ channels: F(4,3) from 256 tiles when 128+ channels come in (128->64@40x40
//    batch 4: 20.8 against 23.3 us), from 512 at 64 channels in (64@56x56 batch 2,
//    392 tiles: 15.0 against 12.3 us on the implicit GEMM; batch 4, 784 tiles: 20.2
//    against 21.7).
//  * fewer channels: the one-launch F(4,3) where it applies (many tiles), else the
//    implicit GEMM.
static int winograd_tile_for(const SpinnHipConvDesc *d) {
    if (wino4_fused_selected(d)) return 4;
    const int64_t t4 = (int64_t)d->n * ((d->oh + 3) / 4) * ((d->ow + 3) / 4);
    if (d->c >= 128 && d->oc >= 128) {
        if (d->c >= 512) return t4 < 16 ? 0 : (t4 < 48 ? 2 : 4);
        return t4 >= (d->c >= 256 ? 64 : 128) ? 4 : 0;
    }
    if (d->c >= 64 && d->oc >= 64) return t4 >= (d->c >= 128 ? 256 : 512) ? 4 : 0;
    return 0;
}

static int select_algo(const SpinnHipConvDesc *d) {
    if (d->algo != SPINN_CONV_ALGO_AUTO) return d->algo;
    const int Cg = d->c / d->group;
    const int OCg = d->oc / d->group;
    if (d->group > 1 && (Cg < 8 || OCg < 8)) return SPINN_CONV_ALGO_DIRECT;
    if (stem_conv_pays(d)) return SPINN_CONV_ALGO_DIRECT;
    if (winograd_eligible(d)) {
        const int w = env_winograd();
        const int fixed = env_winograd_tile();
        int m = w == 0 ? 0 : winograd_tile_for(d);
        if (w == 1 && m == 0) m = 4;
        if (m && fixed) m = fixed;
        if (m) return m == 4 ? SPINN_CONV_ALGO_WINOGRAD_F43 : SPINN_CONV_ALGO_WINOGRAD;
    }
    return SPINN_CONV_ALGO_IMPLICIT_GEMM;
}

static bool conv_desc_ok(const SpinnHipConvDesc *d) {
    if (!d) return false;
    if (d->n <= 0 || d->c <= 0 || d->h <= 0 || d->w <= 0 || d->oc <= 0 || d->oh <= 0 || d->ow <= 0) return false;
    if (d->kh <= 0 || d->kw <= 0 || d->sh <= 0 || d->sw <= 0 || d->ph < 0 || d->pw < 0) return false;
    if (d->group <= 0 || d->c % d->group != 0 || d->oc % d->group != 0) return false;
    if (d->act < 0 || d->act > 5) return false;
    // 32-bit tile indexing: pixels per launch and elements per image plane
    const int64_t ntot = (int64_t)d->n * d->oh * d->ow;
    if (ntot > (int64_t)INT32_MAX || (int64_t)d->c * d->kh * d->kw > (int64_t)INT32_MAX) return false;
    return true;
}

} // namespace spinn

using namespace spinn;

extern "C" {

int spinn_hip_conv_select_algo(const SpinnHipConvDesc *d) {
    if (!conv_desc_ok(d)) return SPINN_HIP_EINVAL;
    return select_algo(d);
}

size_t spinn_hip_conv_workspace_size(const SpinnHipConvDesc *d) {
    if (!conv_desc_ok(d)) return 0;
    switch (select_algo(d)) {
    case SPINN_CONV_ALGO_IMPLICIT_GEMM: return igemm_workspace_bytes(d);
    case SPINN_CONV_ALGO_WINOGRAD: return winograd_eligible(d) ? winograd_workspace_bytes(d, 2) : 0;
    case SPINN_CONV_ALGO_WINOGRAD_F43: return winograd_eligible(d) ? winograd_workspace_bytes(d, 4) : 0;
    default: return 0;
    }
}

size_t spinn_hip_conv_packed_size(const SpinnHipConvDesc *d) {
    if (!conv_desc_ok(d)) return 0;
    switch (select_algo(d)) {
    case SPINN_CONV_ALGO_IMPLICIT_GEMM: return (size_t)igemm_packed_floats(d) * sizeof(float);
    case SPINN_CONV_ALGO_WINOGRAD:
        return winograd_eligible(d) ? (size_t)winograd_packed_floats(d, 2) * sizeof(float) : 0;
    case SPINN_CONV_ALGO_WINOGRAD_F43:
        return winograd_eligible(d) ? (size_t)winograd_packed_floats(d, 4) * sizeof(float) : 0;
    default: return 0;
    }
}

int spinn_hip_conv_pack_weights(const SpinnHipConvDesc *d, const float *w, float *packed, void *stream) {
    if (!conv_desc_ok(d) || !w || !packed) return SPINN_HIP_EINVAL;
    hipStream_t st = (hipStream_t)stream;
    const int algo = select_algo(d);
    switch (algo) {
    case SPINN_CONV_ALGO_IMPLICIT_GEMM: return igemm_pack(d, w, packed, st);
    case SPINN_CONV_ALGO_WINOGRAD:
    case SPINN_CONV_ALGO_WINOGRAD_F43:
        if (!winograd_eligible(d)) return SPINN_HIP_EUNSUPPORTED;
        return winograd_pack(d, algo == SPINN_CONV_ALGO_WINOGRAD ? 2 : 4, w, packed, st);
    default: return SPINN_HIP_OK; // reads w directly
    }
}

int spinn_hip_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed_w,
                   const float *bias, const float *residual, float *y, void *workspace, size_t workspace_bytes,
                   void *stream) {
    if (!conv_desc_ok(d) || !x || !y) return SPINN_HIP_EINVAL;
    const bool has_res = d->act == SPINN_ACT_ADD || d->act == SPINN_ACT_ADD_RELU;
    if (has_res != (residual != nullptr)) return SPINN_HIP_EINVAL;
    hipStream_t st = (hipStream_t)stream;
    const int algo = select_algo(d);
    switch (algo) {
    case SPINN_CONV_ALGO_IMPLICIT_GEMM:
        if (!packed_w) return SPINN_HIP_EINVAL;
        return igemm_conv(d, x, w, packed_w, bias, residual, y, workspace, workspace_bytes, st);
    case SPINN_CONV_ALGO_WINOGRAD:
    case SPINN_CONV_ALGO_WINOGRAD_F43:
        if (!winograd_eligible(d)) return SPINN_HIP_EUNSUPPORTED;
        if (!packed_w) return SPINN_HIP_EINVAL;
        return winograd_conv(d, algo == SPINN_CONV_ALGO_WINOGRAD ? 2 : 4, x, packed_w, bias, residual, y,
                             workspace, workspace_bytes, st);
    case SPINN_CONV_ALGO_DIRECT:
        if (!w) return SPINN_HIP_EINVAL;
        return direct_conv(d, x, w, bias, residual, y, st);
    default: return SPINN_HIP_EINVAL;
    }
}

static bool gemm_desc_ok(const SpinnHipGemmDesc *d) {
    if (!d) return false;
    if (d->m <= 0 || d->n <= 0 || d->k <= 0) return false;
    if (d->c_mode < 0 || d->c_mode > 2) return false;
    if (d->batch < 0) return false;
    if (d->batch > 1 && (d->stride_a < 0 || d->stride_b < 0 || d->stride_y <= 0)) return false;
    return true;
}

size_t spinn_hip_gemm_workspace_size(const SpinnHipGemmDesc *d) {
    if (!gemm_desc_ok(d)) return 0;
    return gemm_workspace_bytes(d);
}

int spinn_hip_gemm(const SpinnHipGemmDesc *d, const float *a, const float *b, const float *c, float *y,
                   void *workspace, size_t workspace_bytes, void *stream) {
    if (!gemm_desc_ok(d) || !a || !b || !y) return SPINN_HIP_EINVAL;
    if (d->c_mode != 0 && !c) return SPINN_HIP_EINVAL;
    return gemm_run(d, a, b, c, y, workspace, workspace_bytes, (hipStream_t)stream);
}

int spinn_hip_maxpool2d(const SpinnHipPoolDesc *d, const float *x, float *y, void *stream) {
    if (!d || !x || !y || d->n <= 0 || d->c <= 0 || d->h <= 0 || d->w <= 0 || d->oh <= 0 || d->ow <= 0 ||
        d->kh <= 0 || d->kw <= 0 || d->sh <= 0 || d->sw <= 0)
        return SPINN_HIP_EINVAL;
    return maxpool2d(d, x, y, (hipStream_t)stream);
}

int spinn_hip_reduce_mean(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, void *stream) {
    if (!x || !y || outer <= 0 || dim <= 0 || inner <= 0) return SPINN_HIP_EINVAL;
    return reduce_mean(outer, dim, inner, x, y, (hipStream_t)stream);
}

int spinn_hip_copy(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0 || dst == src) return SPINN_HIP_OK;
    if (!dst || !src) return SPINN_HIP_EINVAL;
    return hip_code(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int spinn_hip_binary(int op, const float *a, int64_t na, const float *b, int64_t nb, float *y, int64_t n,
                     void *stream) {
    constexpr int64_t kMax = (int64_t)UINT32_MAX;
    if (op < SPINN_BINARY_ADD || op > SPINN_BINARY_DIV || n < 0 || n > kMax || na > kMax || nb > kMax)
        return SPINN_HIP_EINVAL;
    if (n == 0) return SPINN_HIP_OK;
    if (!a || !b || !y || na <= 0 || nb <= 0) return SPINN_HIP_EINVAL;
    return binary_op(op, a, na, b, nb, y, n, (hipStream_t)stream);
}

int spinn_hip_unary(int op, const float *x, float *y, int64_t n, void *stream) {
    if (op < SPINN_UNARY_RELU || op > SPINN_UNARY_SILU || n < 0) return SPINN_HIP_EINVAL;
    if (n == 0) return SPINN_HIP_OK;
    if (!x || !y) return SPINN_HIP_EINVAL;
    return unary_op(op, x, y, n, (hipStream_t)stream);
}

int spinn_hip_batchnorm(int64_t n, int64_t c, int64_t spatial, const float *x, const float *scale,
                        const float *bias, const float *mean, const float *var, float eps, float *y,
                        void *stream) {
    if (n < 0 || c < 0 || spatial < 0) return SPINN_HIP_EINVAL;
    if (n * c * spatial == 0) return SPINN_HIP_OK;
    if (!x || !scale || !bias || !mean || !var || !y) return SPINN_HIP_EINVAL;
    return batchnorm(n, c, spatial, x, scale, bias, mean, var, eps, y, (hipStream_t)stream);
}

int spinn_hip_softmax(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, void *stream) {
    if (outer < 0 || dim < 0 || inner < 0) return SPINN_HIP_EINVAL;
    if (outer * dim * inner == 0) return SPINN_HIP_OK;
    if (!x || !y) return SPINN_HIP_EINVAL;
    return softmax(outer, dim, inner, x, y, (hipStream_t)stream);
}

int spinn_hip_block_copy(const SpinnHipBlockCopy *blocks, int n_blocks, int64_t outer, void *stream) {
    if (!blocks || n_blocks < 0 || n_blocks > SPINN_HIP_MAX_BLOCKS || outer < 0) return SPINN_HIP_EINVAL;
    for (int i = 0; i < n_blocks; ++i) {
        const SpinnHipBlockCopy &b = blocks[i];
        if (b.len < 0 || b.src_row < 0 || b.dst_row < 0 || b.src_off < 0 || b.dst_off < 0) return SPINN_HIP_EINVAL;
        if (b.len > 0 && outer > 0 && (!b.src || !b.dst)) return SPINN_HIP_EINVAL;
    }
    return block_copy(blocks, n_blocks, outer, (hipStream_t)stream);
}

int spinn_hip_transpose(int ndim, const int64_t *dims, const int32_t *perm, const float *x, float *y,
                        void *stream) {
    if (ndim < 1 || ndim > 8 || !dims) return SPINN_HIP_EINVAL;
    int64_t total = 1;
    unsigned seen = 0;
    for (int d = 0; d < ndim; ++d) {
        if (dims[d] < 0) return SPINN_HIP_EINVAL;
        total *= dims[d];
        if (perm) {
            if (perm[d] < 0 || perm[d] >= ndim || (seen >> perm[d] & 1u)) return SPINN_HIP_EINVAL;
            seen |= 1u << perm[d];
        }
    }
    if (total == 0) return SPINN_HIP_OK;
    if (!x || !y || total > (int64_t)UINT32_MAX) return SPINN_HIP_EINVAL;
    return transpose(ndim, dims, perm, x, y, (hipStream_t)stream);
}

int spinn_hip_resize_nearest(int64_t nc, int32_t h, int32_t w, int32_t oh, int32_t ow, const float *x, float *y,
                             void *stream) {
    if (nc < 0 || h <= 0 || w <= 0 || oh < 0 || ow < 0) return SPINN_HIP_EINVAL;
    if (nc * oh * ow == 0) return SPINN_HIP_OK;
    if (!x || !y) return SPINN_HIP_EINVAL;
    return resize_nearest(nc, h, w, oh, ow, x, y, (hipStream_t)stream);
}

int spinn_hip_reduce_max(int64_t rows, int64_t block, const float *x, float *y, void *stream) {
    if (rows < 0 || block < 0) return SPINN_HIP_EINVAL;
    if (rows == 0) return SPINN_HIP_OK;
    if (!x || !y || block == 0 || rows > (int64_t)UINT32_MAX * 4) return SPINN_HIP_EINVAL;
    return reduce_max_rows(rows, block, x, y, (hipStream_t)stream);
}

int spinn_hip_topk(int64_t rows, int64_t n, int64_t k, const float *x, float *values, int64_t *indices,
                   void *stream) {
    if (rows < 0 || n < 0 || k < 0) return SPINN_HIP_EINVAL;
    if (rows == 0 || k == 0) return SPINN_HIP_OK;
    if (k > n || n >= (int64_t)INT32_MAX || rows > (int64_t)UINT32_MAX) return SPINN_HIP_EINVAL;
    if (k > SPINN_HIP_TOPK_MAX_K) return SPINN_HIP_EUNSUPPORTED;
    if (!x || !values || !indices) return SPINN_HIP_EINVAL;
    return topk_rows(rows, n, (int)k, x, values, indices, (hipStream_t)stream);
}

int spinn_hip_gather_elements(const SpinnHipGatherDesc *d, const float *data, const void *indices, float *y,
                              void *stream) {
    if (!d || d->ndim < 1 || d->ndim > 8 || d->axis < 0 || d->axis >= d->ndim) return SPINN_HIP_EINVAL;
    if (d->index_dtype != ENNF_TYPE_INT64 && d->index_dtype != ENNF_TYPE_INT32) return SPINN_HIP_EINVAL;
    int64_t total = 1;
    for (int i = 0; i < d->ndim; ++i) {
        if (d->in_dims[i] < 0 || d->out_dims[i] < 0) return SPINN_HIP_EINVAL;
        // outside the gathered axis the indices may not reach past the data (ONNX rule)
        if (i != d->axis && d->out_dims[i] > d->in_dims[i]) return SPINN_HIP_EINVAL;
        total *= d->out_dims[i];
    }
    if (total == 0) return SPINN_HIP_OK;
    if (d->in_dims[d->axis] == 0 || !data || !indices || !y) return SPINN_HIP_EINVAL;
    return gather_elements(d, data, indices, y, (hipStream_t)stream);
}

int spinn_hip_tile(int ndim, const int64_t *in_dims, const int64_t *out_dims, int elem_bytes, const void *x,
                   void *y, void *stream) {
    if (ndim < 1 || ndim > 8 || !in_dims || !out_dims) return SPINN_HIP_EINVAL;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return SPINN_HIP_EINVAL;
    int64_t total = 1;
    for (int i = 0; i < ndim; ++i) {
        if (in_dims[i] < 0 || out_dims[i] < 0) return SPINN_HIP_EINVAL;
        if (out_dims[i] > 0 && in_dims[i] == 0) return SPINN_HIP_EINVAL;
        total *= out_dims[i];
    }
    if (total == 0) return SPINN_HIP_OK;
    if (!x || !y) return SPINN_HIP_EINVAL;
    return tile(ndim, in_dims, out_dims, elem_bytes, x, y, (hipStream_t)stream);
}

int spinn_hip_cast(int src_dtype, int dst_dtype, int64_t n, const void *x, void *y, void *stream) {
    auto known = [](int t) { return t == ENNF_TYPE_FLOAT32 || t == ENNF_TYPE_INT32 || t == ENNF_TYPE_INT64; };
    if (n < 0) return SPINN_HIP_EINVAL;
    if (!known(src_dtype) || !known(dst_dtype)) return SPINN_HIP_EUNSUPPORTED;
    if (n == 0) return SPINN_HIP_OK;
    if (!x || !y) return SPINN_HIP_EINVAL;
    return cast(src_dtype, dst_dtype, n, x, y, (hipStream_t)stream);
}

int spinn_hip_binary_typed(int op, int dtype, const void *a, int64_t na, const void *b, int64_t nb, void *y,
                           int64_t n, void *stream) {
    constexpr int64_t kMax = (int64_t)UINT32_MAX;
    if (op < SPINN_BINARY_ADD || op > SPINN_BINARY_MOD || n < 0 || n > kMax || na > kMax || nb > kMax)
        return SPINN_HIP_EINVAL;
    if (dtype != ENNF_TYPE_FLOAT32 && dtype != ENNF_TYPE_INT32 && dtype != ENNF_TYPE_INT64)
        return SPINN_HIP_EUNSUPPORTED;
    if (n == 0) return SPINN_HIP_OK;
    if (!a || !b || !y || na <= 0 || nb <= 0) return SPINN_HIP_EINVAL;
    return binary_typed(op, dtype, a, na, b, nb, y, n, (hipStream_t)stream);
}

int spinn_hip_init(int device) {
    int rc = hip_code(hipSetDevice(device));
    if (rc) return rc;
    // resolve the device address of spinn_hip_conv_noalloc's scratch array here,
    // at set-up, rather than inside a caller's capture or serving loop
    void *scratch = nullptr;
    rc = noalloc_scratch(device, &scratch);
    if (rc) return rc;
    probe_xcd_local(device);
    init_device_status();
    return SPINN_HIP_OK;
}

int spinn_hip_device_status(void) { return take_device_status() ? SPINN_HIP_EDEVICE : SPINN_HIP_OK; }

int spinn_hip_device_count(int *count) {
    if (!count) return SPINN_HIP_EINVAL;
    return hip_code(hipGetDeviceCount(count));
}

int spinn_hip_malloc(void **ptr, size_t bytes) {
    if (!ptr) return SPINN_HIP_EINVAL;
    *ptr = nullptr;
    if (bytes == 0) return SPINN_HIP_OK;
    return hip_code(hipMalloc(ptr, bytes));
}

int spinn_hip_free(void *ptr) { return ptr ? hip_code(hipFree(ptr)) : SPINN_HIP_OK; }

int spinn_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return SPINN_HIP_OK;
    if (!dst || !src) return SPINN_HIP_EINVAL;
    return hip_code(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
}

int spinn_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return SPINN_HIP_OK;
    if (!dst || !src) return SPINN_HIP_EINVAL;
    return hip_code(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
}

int spinn_hip_fill_u32(void *dst, uint32_t value, size_t bytes, void *stream) {
    if (bytes % 4 != 0) return SPINN_HIP_EINVAL;
    if (bytes == 0) return SPINN_HIP_OK;
    if (!dst) return SPINN_HIP_EINVAL;
    return fill_u32(dst, value, bytes, (hipStream_t)stream);
}

int spinn_hip_stream_create(void **stream) {
    if (!stream) return SPINN_HIP_EINVAL;
    hipStream_t s = nullptr;
    int rc = hip_code(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = rc ? nullptr : (void *)s;
    return rc;
}

int spinn_hip_stream_destroy(void *stream) {
    return stream ? hip_code(hipStreamDestroy((hipStream_t)stream)) : SPINN_HIP_OK;
}

int spinn_hip_stream_sync(void *stream) { return hip_code(hipStreamSynchronize((hipStream_t)stream)); }

int spinn_hip_event_create(void **event) {
    if (!event) return SPINN_HIP_EINVAL;
    hipEvent_t e = nullptr;
    int rc = hip_code(hipEventCreate(&e));
    *event = rc ? nullptr : (void *)e;
    return rc;
}

int spinn_hip_event_destroy(void *event) {
    return event ? hip_code(hipEventDestroy((hipEvent_t)event)) : SPINN_HIP_OK;
}

int spinn_hip_event_record(void *event, void *stream) {
    if (!event) return SPINN_HIP_EINVAL;
    return hip_code(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
}

int spinn_hip_event_elapsed_ms(void *start, void *stop, float *ms) {
    if (!start || !stop || !ms) return SPINN_HIP_EINVAL;
    int rc = hip_code(hipEventSynchronize((hipEvent_t)stop));
    if (rc) return rc;
    return hip_code(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}

int spinn_hip_graph_capture_begin(void *stream) {
    if (!stream) return SPINN_HIP_EINVAL; // the null stream cannot be captured
    return hip_code(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
}

int spinn_hip_graph_capture_end(void *stream, void **graph_exec) {
    if (!stream || !graph_exec) return SPINN_HIP_EINVAL;
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    int rc = hip_code(hipStreamEndCapture((hipStream_t)stream, &g));
    if (rc) return rc;
    hipGraphExec_t ex = nullptr;
    rc = hip_code(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *graph_exec = (void *)ex;
    return SPINN_HIP_OK;
}

int spinn_hip_graph_launch(void *graph_exec, void *stream) {
    if (!graph_exec) return SPINN_HIP_EINVAL;
    return hip_code(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream));
}

int spinn_hip_graph_destroy(void *graph_exec) {
    return graph_exec ? hip_code(hipGraphExecDestroy((hipGraphExec_t)graph_exec)) : SPINN_HIP_OK;
}

const char *spinn_hip_error_string(int code) {
    if (code == SPINN_HIP_OK) return "ok";
    if (code == SPINN_HIP_EINVAL) return "invalid argument";
    if (code == SPINN_HIP_EUNSUPPORTED) return "unsupported configuration";
    if (code == SPINN_HIP_EWORKSPACE) return "workspace missing or too small";
    if (code == SPINN_HIP_EDEVICE) return "a kernel reported an internal failure (stream-K tile left unfinished)";
    if (code <= SPINN_HIP_ERUNTIME) return hipGetErrorString((hipError_t)(SPINN_HIP_ERUNTIME - code));
    return "unknown error";
}

void spinn_hip_tune_force_tiles(int bm, int bn, int split) { force_tiles(bm, bn, split); }

void spinn_hip_tune_streamk(int mode) { force_streamk(mode); }

void spinn_hip_tune_streamk_tries(int tries) { force_streamk_tries(tries); }

void spinn_hip_tune_winograd_fused(int mode) { force_winograd_fused(mode); }

const char *spinn_hip_version(void) { return "spinn_amd 0.1 gfx950 fp32-mfma"; }

} // extern "C"
