/* hip_stub.c - host-memory stand-in for the device layer (include/spinn_hip.h),
 * for a CPU build of the C runtime under AddressSanitizer / UBSan.
 *
 * Test infrastructure only: it lets the loader, the planner and every
 * operator's host-side operand reading (spinn_amd/csrc/host/) run on a machine
 * without a GPU, so the sanitizers see every byte the host code touches while
 * it parses an untrusted .ennf file. "Device" memory is host memory from
 * malloc, copies are memcpy, compute entry points validate nothing and do no
 * arithmetic (they return 0 so the node loop reaches every node). Graph
 * capture reports an error, so graph mode falls back to its error path.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include "spinn_hip.h"

int spinn_hip_init(int device) { (void)device; return 0; }
int spinn_hip_device_count(int *count) { *count = 1; return 0; }
int spinn_hip_malloc(void **ptr, size_t bytes) {
    *ptr = malloc(bytes ? bytes : 1);
    return *ptr ? 0 : SPINN_HIP_ERUNTIME - 2;
}
int spinn_hip_free(void *ptr) { free(ptr); return 0; }
int spinn_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    (void)stream;
    if (bytes) memcpy(dst, src, bytes);
    return 0;
}
int spinn_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    (void)stream;
    if (bytes) memcpy(dst, src, bytes);
    return 0;
}
int spinn_hip_copy(void *dst, const void *src, size_t bytes, void *stream) {
    (void)stream;
    if (bytes) memmove(dst, src, bytes);
    return 0;
}
int spinn_hip_device_status(void) { return 0; }
int spinn_hip_fill_u32(void *dst, uint32_t value, size_t bytes, void *stream) {
    (void)stream;
    uint32_t *p = (uint32_t *)dst;
    for (size_t i = 0; i < bytes / 4; i++) p[i] = value;
    return 0;
}
static int g_stream_token, g_event_token;
int spinn_hip_stream_create(void **stream) { *stream = &g_stream_token; return 0; }
int spinn_hip_stream_destroy(void *stream) { (void)stream; return 0; }
int spinn_hip_stream_sync(void *stream) { (void)stream; return 0; }
int spinn_hip_event_create(void **event) { *event = &g_event_token; return 0; }
int spinn_hip_event_destroy(void *event) { (void)event; return 0; }
int spinn_hip_event_record(void *event, void *stream) { (void)event; (void)stream; return 0; }
int spinn_hip_event_elapsed_ms(void *start, void *stop, float *ms) {
    (void)start; (void)stop;
    *ms = 0.f;
    return 0;
}
int spinn_hip_graph_capture_begin(void *stream) { (void)stream; return SPINN_HIP_EUNSUPPORTED; }
int spinn_hip_graph_capture_end(void *stream, void **graph_exec) {
    (void)stream;
    *graph_exec = NULL;
    return SPINN_HIP_EUNSUPPORTED;
}
int spinn_hip_graph_launch(void *graph_exec, void *stream) { (void)graph_exec; (void)stream; return SPINN_HIP_EUNSUPPORTED; }
int spinn_hip_graph_destroy(void *graph_exec) { (void)graph_exec; return 0; }
const char *spinn_hip_error_string(int code) { (void)code; return "host stub"; }

/* Conv: the implicit-GEMM layout sizes (W^T [K][OC rounded to 4]) so the
 * planner's packed-weight pool and the prepare pass run as on the GPU. */
int spinn_hip_conv_select_algo(const SpinnHipConvDesc *d) { (void)d; return SPINN_CONV_ALGO_IMPLICIT_GEMM; }
size_t spinn_hip_conv_workspace_size(const SpinnHipConvDesc *d) { (void)d; return 0; }
size_t spinn_hip_conv_packed_size(const SpinnHipConvDesc *d) {
    if (d->group <= 0 || d->group > 1) return 0;
    return (size_t)d->c * d->kh * d->kw * (size_t)((d->oc + 3) / 4 * 4) * sizeof(float);
}
int spinn_hip_conv_pack_weights(const SpinnHipConvDesc *d, const float *w, float *packed, void *stream) {
    (void)stream;
    size_t n = spinn_hip_conv_packed_size(d) / sizeof(float);
    size_t nw = (size_t)d->oc * d->c * d->kh * d->kw;
    for (size_t i = 0; i < n; i++) packed[i] = w[i % nw];
    return 0;
}
int spinn_hip_conv(const SpinnHipConvDesc *d, const float *x, const float *w, const float *packed_w,
                   const float *bias, const float *residual, float *y, void *workspace, size_t workspace_bytes,
                   void *stream) {
    (void)d; (void)x; (void)w; (void)packed_w; (void)bias; (void)residual; (void)y; (void)workspace;
    (void)workspace_bytes; (void)stream;
    return 0;
}
int spinn_hip_gemm(const SpinnHipGemmDesc *d, const float *a, const float *b, const float *c, float *y,
                   void *workspace, size_t workspace_bytes, void *stream) {
    (void)d; (void)a; (void)b; (void)c; (void)y; (void)workspace; (void)workspace_bytes; (void)stream;
    return 0;
}
size_t spinn_hip_gemm_workspace_size(const SpinnHipGemmDesc *d) { (void)d; return 0; }
int spinn_hip_maxpool2d(const SpinnHipPoolDesc *d, const float *x, float *y, void *stream) {
    (void)d; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_reduce_mean(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, void *stream) {
    (void)outer; (void)dim; (void)inner; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_binary(int op, const float *a, int64_t na, const float *b, int64_t nb, float *y, int64_t n,
                     void *stream) {
    (void)op; (void)a; (void)na; (void)b; (void)nb; (void)y; (void)n; (void)stream;
    return 0;
}
int spinn_hip_unary(int op, const float *x, float *y, int64_t n, void *stream) {
    (void)op; (void)x; (void)y; (void)n; (void)stream;
    return 0;
}
int spinn_hip_batchnorm(int64_t n, int64_t c, int64_t spatial, const float *x, const float *scale,
                        const float *bias, const float *mean, const float *var, float eps, float *y, void *stream) {
    (void)n; (void)c; (void)spatial; (void)x; (void)scale; (void)bias; (void)mean; (void)var; (void)eps; (void)y;
    (void)stream;
    return 0;
}
int spinn_hip_softmax(int64_t outer, int64_t dim, int64_t inner, const float *x, float *y, void *stream) {
    (void)outer; (void)dim; (void)inner; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_block_copy(const SpinnHipBlockCopy *blocks, int n_blocks, int64_t outer, void *stream) {
    (void)blocks; (void)n_blocks; (void)outer; (void)stream;
    return 0;
}
int spinn_hip_transpose(int ndim, const int64_t *dims, const int32_t *perm, const float *x, float *y,
                        void *stream) {
    (void)ndim; (void)dims; (void)perm; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_resize_nearest(int64_t nc, int32_t h, int32_t w, int32_t oh, int32_t ow, const float *x, float *y,
                             void *stream) {
    (void)nc; (void)h; (void)w; (void)oh; (void)ow; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_reduce_max(int64_t rows, int64_t block, const float *x, float *y, void *stream) {
    (void)rows; (void)block; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_topk(int64_t rows, int64_t n, int64_t k, const float *x, float *values, int64_t *indices,
                   void *stream) {
    (void)rows; (void)n; (void)k; (void)x; (void)values; (void)indices; (void)stream;
    return 0;
}
int spinn_hip_gather_elements(const SpinnHipGatherDesc *d, const float *data, const void *indices, float *y,
                              void *stream) {
    (void)d; (void)data; (void)indices; (void)y; (void)stream;
    return 0;
}
int spinn_hip_tile(int ndim, const int64_t *in_dims, const int64_t *out_dims, int elem_bytes, const void *x,
                   void *y, void *stream) {
    (void)ndim; (void)in_dims; (void)out_dims; (void)elem_bytes; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_cast(int src_dtype, int dst_dtype, int64_t n, const void *x, void *y, void *stream) {
    (void)src_dtype; (void)dst_dtype; (void)n; (void)x; (void)y; (void)stream;
    return 0;
}
int spinn_hip_binary_typed(int op, int dtype, const void *a, int64_t na, const void *b, int64_t nb, void *y,
                           int64_t n, void *stream) {
    (void)op; (void)dtype; (void)a; (void)na; (void)b; (void)nb; (void)y; (void)n; (void)stream;
    return 0;
}
