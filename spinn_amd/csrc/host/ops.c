/*
 * ops.c - operator registry and the device operator kernels behind it.
 *
 * The registry and dispatcher keep the reference's contract
 * (SPINN/run_time/spinn_ops.c:17-228): a lazily filled table of 512
 * SpinnOpKernel slots indexed by ENNF op id; an id >= 512 returns -1; an
 * unregistered op prints a notice and returns 0 (skipped).
 *
 * Each kernel reads its operands exactly as the reference operator does
 * (arity, dims, params, fused-act sniffing), then hands device pointers to the
 * HIP C ABI (spinn_hip_*). Nothing here touches tensor data on the host.
 */
#include "spinn_host.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

SpinnExec g_spinn_exec = {.matmul_alpha = 1.f};

static void *g_fallback_ws = NULL;
static size_t g_fallback_ws_bytes = 0;

void *spinn_exec_workspace(size_t bytes) {
    if (bytes == 0) return NULL;
    if (g_spinn_exec.workspace && g_spinn_exec.workspace_bytes >= bytes) return g_spinn_exec.workspace;
    if (g_fallback_ws_bytes < bytes) {
        if (g_fallback_ws) spinn_hip_free(g_fallback_ws);
        g_fallback_ws = NULL;
        g_fallback_ws_bytes = 0;
        if (spinn_hip_malloc(&g_fallback_ws, bytes) != 0) return NULL;
        g_fallback_ws_bytes = bytes;
    }
    return g_fallback_ws;
}

void spinn_exec_release_fallback(void) {
    if (g_fallback_ws) spinn_hip_free(g_fallback_ws);
    g_fallback_ws = NULL;
    g_fallback_ws_bytes = 0;
}

/* Packed-weight buffers: device payload plus a host record of (algo, bytes). */
typedef struct PackedRec {
    void *dev;
    size_t bytes;
    int algo;
    struct PackedRec *next;
} PackedRec;
static PackedRec *g_packed = NULL;

int spinn_packed_alloc(void **dev, size_t bytes, int algo) {
    PackedRec *r = (PackedRec *)calloc(1, sizeof(PackedRec));
    if (!r) return -1;
    int rc = spinn_hip_malloc(&r->dev, bytes);
    if (rc) {
        free(r);
        return rc;
    }
    r->bytes = bytes;
    r->algo = algo;
    r->next = g_packed;
    g_packed = r;
    *dev = r->dev;
    return 0;
}

int spinn_packed_matches(const void *dev, size_t bytes, int algo) {
    for (PackedRec *r = g_packed; r; r = r->next)
        if (r->dev == dev) return r->bytes == bytes && r->algo == algo;
    return 0;
}

void spinn_packed_release(void *dev) {
    PackedRec **pp = &g_packed;
    while (*pp) {
        if ((*pp)->dev == dev) {
            PackedRec *r = *pp;
            *pp = r->next;
            spinn_hip_free(r->dev);
            free(r);
            return;
        }
        pp = &(*pp)->next;
    }
}

static void note_workspace(size_t need) {
    if (need > g_spinn_exec.prepare_ws_need) g_spinn_exec.prepare_ws_need = need;
}

/* A float32 operand holding exactly `elems` elements with device memory behind
 * it. The loader already holds elem_count to the product of the dims and size
 * to elem_count * 4, so this ties a kernel's extents to the buffer it gets. */
static int f32_operand(const SpinnTensor *t, uint64_t elems) {
    return t && t->data && t->dtype == ENNF_TYPE_FLOAT32 && elems > 0 && (uint64_t)t->elem_count == elems;
}

/* ------------------------------------------------------------------------
 * Conv (SPINN/run_time/ops/conv/conv2d.c:92-232)
 * ---------------------------------------------------------------------- */
int spinn_conv_desc_from_tensors(SpinnTensor **in, int n_in, const void *params, uint16_t params_size,
                                 SpinnTensor **out, SpinnHipConvDesc *d, const float **bias, const float **res) {
    if (n_in < 2 || !out || !out[0]) return -1;
    const ENNF_ConvParams *p =
        (params && params_size >= sizeof(ENNF_ConvParams)) ? (const ENNF_ConvParams *)params : NULL;
    /* The act code is read before the inputs: with ADD / ADD_RELU the last
     * input is the residual, not a bias (conv2d.c:96-105). */
    const int act = p ? p->reserved : 0;
    const int has_res = (act == SPINN_ACT_ADD || act == SPINN_ACT_ADD_RELU);
    const int n_real = has_res ? n_in - 1 : n_in;
    if (has_res && n_in < 3) return -1;
    SpinnTensor *X = in[0], *W = in[1], *Y = out[0];
    if (!X || !W || X->ndim != 4 || W->ndim != 4 || Y->ndim != 4) return -1;
    memset(d, 0, sizeof(*d));
    d->n = (int)X->dims[0];
    d->c = (int)X->dims[1];
    d->h = (int)X->dims[2];
    d->w = (int)X->dims[3];
    d->oc = (int)W->dims[0];
    const int kc = (int)W->dims[1];
    d->kh = (int)W->dims[2];
    d->kw = (int)W->dims[3];
    d->sh = d->sw = 1;
    d->group = 1;
    d->oh = (int)Y->dims[2];
    d->ow = (int)Y->dims[3];
    if (p) {
        if (p->group > 0) d->group = p->group;
        if (p->kernel_shape[0] > 0) d->kh = p->kernel_shape[0];
        if (p->kernel_shape[1] > 0) d->kw = p->kernel_shape[1];
        if (p->strides[0] > 0) d->sh = p->strides[0];
        if (p->strides[1] > 0) d->sw = p->strides[1];
        /* Only the begin pads are used; dilations are ignored (conv2d.c:131). */
        d->ph = p->pads[0];
        d->pw = p->pads[1];
        if (p->auto_pad == ENNF_AUTOPAD_SAME_UPPER || p->auto_pad == ENNF_AUTOPAD_SAME_LOWER) {
            int ph = (d->oh - 1) * d->sh + d->kh - d->h;
            int pw = (d->ow - 1) * d->sw + d->kw - d->w;
            if (ph < 0) ph = 0;
            if (pw < 0) pw = 0;
            d->ph = (p->auto_pad == ENNF_AUTOPAD_SAME_UPPER) ? ph / 2 : (ph + 1) / 2;
            d->pw = (p->auto_pad == ENNF_AUTOPAD_SAME_UPPER) ? pw / 2 : (pw + 1) / 2;
        }
    }
    d->act = act;
    if (kc * d->group != d->c || (int)Y->dims[1] != d->oc || (int)Y->dims[0] != d->n) return -1;
    /* The kernels size every read and write from the descriptor: the window must
     * be the weight tensor's own (params cannot widen it), output channels must
     * split evenly over the groups, and each operand must hold what the
     * descriptor says it does. */
    if (d->kh != (int)W->dims[2] || d->kw != (int)W->dims[3] || d->group <= 0 || d->oc % d->group) return -1;
    if (d->n <= 0 || d->c <= 0 || d->h <= 0 || d->w <= 0 || d->oh <= 0 || d->ow <= 0 || d->ph < 0 || d->pw < 0)
        return -1;
    const uint64_t y_elems = (uint64_t)d->n * d->oc * d->oh * d->ow;
    if (!f32_operand(X, (uint64_t)d->n * d->c * d->h * d->w) || !f32_operand(W, (uint64_t)d->oc * kc * d->kh * d->kw) ||
        !f32_operand(Y, y_elems))
        return -1;
    d->algo = SPINN_CONV_ALGO_AUTO;
    int algo = spinn_hip_conv_select_algo(d);
    if (algo < 0) return -1;
    const int wino = algo == SPINN_CONV_ALGO_WINOGRAD || algo == SPINN_CONV_ALGO_WINOGRAD_F43;
    if (wino && g_spinn_exec.conv_policy == SPINN_CONV_POLICY_IGEMM) {
        algo = SPINN_CONV_ALGO_IMPLICIT_GEMM;
    } else if (algo == SPINN_CONV_ALGO_IMPLICIT_GEMM && g_spinn_exec.conv_policy == SPINN_CONV_POLICY_WINOGRAD) {
        d->algo = SPINN_CONV_ALGO_WINOGRAD_F43;
        if (spinn_hip_conv_packed_size(d) == 0) algo = SPINN_CONV_ALGO_IMPLICIT_GEMM; /* not eligible */
        else algo = SPINN_CONV_ALGO_WINOGRAD_F43;
    }
    d->algo = algo;
    *bias = (n_real > 2 && in[2] && in[2]->data) ? (const float *)in[2]->data : NULL;
    *res = has_res ? (const float *)in[n_in - 1]->data : NULL;
    if (has_res && !*res) return -1;
    if (*bias && (in[2]->dtype != ENNF_TYPE_FLOAT32 || in[2]->elem_count < (uint32_t)d->oc)) return -1;
    if (has_res && !f32_operand(in[n_in - 1], y_elems)) return -1;
    return 0;
}

int op_conv2d(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 2 || n_out < 1) return -1;
    SpinnHipConvDesc d;
    const float *bias = NULL, *res = NULL;
    if (spinn_conv_desc_from_tensors(in, n_in, params, params_size, out, &d, &bias, &res) != 0) return -1;
    SpinnTensor *W = in[1];
    /* Weights re-laid out once per tensor and cached on it, like the
     * reference's lazily packed A (conv2d.c:200-207); normally done by the
     * prepare pass of spinn_plan so no run ever allocates. The buffer keeps a
     * host-side record of the layout it holds; a conv that would read it as
     * another layout fails instead of reading past it. */
    const size_t psz = spinn_hip_conv_packed_size(&d);
    if (psz > 0) {
        if (!W->packed_data) {
            void *pk = NULL;
            int rc = spinn_packed_alloc(&pk, psz, d.algo);
            if (rc) return rc;
            rc = spinn_hip_conv_pack_weights(&d, (const float *)W->data, (float *)pk, g_spinn_exec.stream);
            if (rc) {
                spinn_packed_release(pk);
                return rc;
            }
            W->packed_data = pk;
        } else if (!spinn_packed_matches(W->packed_data, psz, d.algo)) {
            return -1;
        }
    }
    const size_t wsz = spinn_hip_conv_workspace_size(&d);
    if (g_spinn_exec.preparing) {
        note_workspace(wsz);
        return 0;
    }
    void *ws = wsz ? spinn_exec_workspace(wsz) : NULL;
    if (wsz && !ws) return SPINN_HIP_EWORKSPACE;
    return spinn_hip_conv(&d, (const float *)in[0]->data, (const float *)W->data, (const float *)W->packed_data,
                          bias, res, (float *)out[0]->data, ws, wsz, g_spinn_exec.stream);
}

/* ------------------------------------------------------------------------
 * Gemm (SPINN/run_time/ops/mm/gemm.c:7-78)
 * ---------------------------------------------------------------------- */
int op_gemm(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 2 || n_out < 1) return -1;
    SpinnTensor *A = in[0], *B = in[1], *Y = out[0];
    SpinnTensor *Cb = (n_in > 2 && in[2] && in[2]->data) ? in[2] : NULL;
    if (A->ndim != 2 || B->ndim != 2) return -1;
    SpinnHipGemmDesc d;
    memset(&d, 0, sizeof(d));
    d.alpha = 1.f;
    d.beta = 1.f;
    if (params && params_size >= sizeof(ENNF_GemmParams)) {
        const ENNF_GemmParams *p = (const ENNF_GemmParams *)params;
        d.trans_a = p->transA;
        d.trans_b = p->transB;
        d.alpha = p->alpha;
        d.beta = p->beta;
    }
    d.m = (int)(d.trans_a ? A->dims[1] : A->dims[0]);
    d.k = (int)(d.trans_a ? A->dims[0] : A->dims[1]);
    d.n = (int)(d.trans_b ? B->dims[0] : B->dims[1]);
    const int kb = (int)(d.trans_b ? B->dims[1] : B->dims[0]);
    if (kb != d.k) return -1;
    if (!f32_operand(A, (uint64_t)d.m * d.k) || !f32_operand(B, (uint64_t)d.k * d.n) ||
        !f32_operand(Y, (uint64_t)d.m * d.n))
        return -1;
    d.batch = 1;
    /* C joins as beta*C only when beta != 0: an [N] vector broadcast over rows,
     * else a full [M,N] matrix (gemm.c:31,62-67). */
    if (Cb && d.beta != 0.0f) {
        if (Cb->dtype != ENNF_TYPE_FLOAT32) return -1;
        if (Cb->elem_count == (uint32_t)d.n) d.c_mode = 1;
        else if (Cb->elem_count == (uint32_t)d.m * (uint32_t)d.n) d.c_mode = 2;
        else return -1;
    }
    const size_t wsz = spinn_hip_gemm_workspace_size(&d);
    if (g_spinn_exec.preparing) {
        note_workspace(wsz);
        return 0;
    }
    void *ws = wsz ? spinn_exec_workspace(wsz) : NULL;
    if (wsz && !ws) return SPINN_HIP_EWORKSPACE;
    return spinn_hip_gemm(&d, (const float *)A->data, (const float *)B->data, d.c_mode ? (const float *)Cb->data : NULL,
                          (float *)Y->data, ws, wsz, g_spinn_exec.stream);
}

/* ------------------------------------------------------------------------
 * MatMul (SPINN/run_time/ops/mm/matmul.c:6-62): 2-D x 2-D, or equal batch
 * products over the leading dims; anything else returns -1 as there.
 * ---------------------------------------------------------------------- */
int op_matmul(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 2 || n_out < 1) return -1;
    SpinnTensor *A = in[0], *B = in[1], *Y = out[0];
    int an = A->ndim, bn = B->ndim;
    if (an < 2 || bn < 2) return -1;
    /* An operand handed over as its transpose (the runtime folded a Transpose of
     * the last two axes into this node) is read with the Gemm's transpose flag. */
    const int ta = g_spinn_exec.matmul_transposed & 1, tb = (g_spinn_exec.matmul_transposed >> 1) & 1;
    SpinnHipGemmDesc d;
    memset(&d, 0, sizeof(d));
    d.alpha = g_spinn_exec.matmul_alpha;
    d.beta = 0.f;
    d.trans_a = ta;
    d.trans_b = tb;
    d.m = (int)A->dims[an - (ta ? 1 : 2)];
    d.k = (int)A->dims[an - (ta ? 2 : 1)];
    d.n = (int)B->dims[bn - (tb ? 2 : 1)];
    if ((int)B->dims[bn - (tb ? 1 : 2)] != d.k) return -1;
    int batch = 1, batch_b = 1;
    for (int i = 0; i < an - 2; i++) batch *= (int)A->dims[i];
    for (int i = 0; i < bn - 2; i++) batch_b *= (int)B->dims[i];
    if (an == 2 && bn == 2) batch = batch_b = 1;
    if (batch != batch_b) return -1;
    if (!f32_operand(A, (uint64_t)batch * d.m * d.k) || !f32_operand(B, (uint64_t)batch * d.k * d.n) ||
        !f32_operand(Y, (uint64_t)batch * d.m * d.n))
        return -1;
    d.batch = batch;
    d.stride_a = (int64_t)d.m * d.k;
    d.stride_b = (int64_t)d.k * d.n;
    d.stride_y = (int64_t)d.m * d.n;
    const size_t wsz = spinn_hip_gemm_workspace_size(&d);
    if (g_spinn_exec.preparing) {
        note_workspace(wsz);
        return 0;
    }
    void *ws = wsz ? spinn_exec_workspace(wsz) : NULL;
    if (wsz && !ws) return SPINN_HIP_EWORKSPACE;
    return spinn_hip_gemm(&d, (const float *)A->data, (const float *)B->data, NULL, (float *)Y->data, ws, wsz,
                          g_spinn_exec.stream);
}

/* ------------------------------------------------------------------------
 * MaxPool (SPINN/run_time/ops/pool/maxpool.c:5-49)
 * ---------------------------------------------------------------------- */
int op_maxpool(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    SpinnTensor *X = in[0], *Y = out[0];
    if (X->ndim != 4 || Y->ndim != 4) return -1;
    SpinnHipPoolDesc d;
    memset(&d, 0, sizeof(d));
    d.n = (int)X->dims[0];
    d.c = (int)X->dims[1];
    d.h = (int)X->dims[2];
    d.w = (int)X->dims[3];
    d.oh = (int)Y->dims[2];
    d.ow = (int)Y->dims[3];
    d.kh = d.kw = d.sh = d.sw = 1;
    if (params && params_size >= sizeof(ENNF_PoolParams)) {
        const ENNF_PoolParams *p = (const ENNF_PoolParams *)params;
        d.kh = p->kernel_shape[0];
        d.kw = p->kernel_shape[1];
        d.sh = p->strides[0];
        d.sw = p->strides[1];
        d.ph = p->pads[0];
        d.pw = p->pads[1];
    }
    if (Y->dims[0] != X->dims[0] || Y->dims[1] != X->dims[1] || !f32_operand(X, X->elem_count) ||
        !f32_operand(Y, Y->elem_count))
        return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_maxpool2d(&d, (const float *)X->data, (float *)Y->data, g_spinn_exec.stream);
}

/* GlobalAveragePool (SPINN/run_time/ops/pool/global_avg_pool.c:4-28). */
int op_global_avg_pool(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out,
                       int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 1 || n_out < 1) return -1;
    SpinnTensor *X = in[0];
    if (X->ndim != 4) return -1;
    if (!f32_operand(X, X->elem_count) || !f32_operand(out[0], (uint64_t)X->dims[0] * X->dims[1])) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_reduce_mean((int64_t)X->dims[0] * X->dims[1], (int64_t)X->dims[2] * X->dims[3], 1,
                                 (const float *)X->data, (float *)out[0]->data, g_spinn_exec.stream);
}

/* ReduceMean: the axis choice of SPINN/run_time/ops/reduce/reduce_mean.c:10-75,
 * then one mean over the middle axis of an [outer, dim, inner] view. */
int op_reduce_mean(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    SpinnTensor *X = in[0], *Y = out[0];
    const ENNF_ReduceParams *p =
        (params && params_size >= sizeof(ENNF_ReduceParams)) ? (const ENNF_ReduceParams *)params : NULL;
    const int ndim = X->ndim;
    int axis = -1, merge = 0;
    if (p && p->num_axes > 0) {
        axis = p->axes[0];
        if (axis < 0) axis += ndim;
        if (p->num_axes > 1 && axis + p->num_axes == ndim) merge = 1;
    }
    if (axis == -1 && (!p || p->num_axes == 0)) {
        if (Y->elem_count > 1 && X->ndim == Y->ndim + 1) {
            int inferred = -1, od = 0;
            for (int dd = 0; dd < X->ndim; dd++) {
                if (od < Y->ndim && X->dims[dd] == Y->dims[od]) od++;
                else if (inferred == -1) inferred = dd;
                else { inferred = -2; break; }
            }
            if (inferred >= 0) axis = inferred;
        } else if (X->ndim == Y->ndim) {
            int first = -1, cnt = 0;
            for (int dd = 0; dd < X->ndim; dd++) {
                if (X->dims[dd] != Y->dims[dd]) {
                    if (Y->dims[dd] == 1) { if (first == -1) first = dd; cnt++; }
                    else { first = -2; break; }
                } else if (first != -1) { first = -2; break; }
            }
            if (first >= 0 && first + cnt == X->ndim) { axis = first; merge = 1; }
        }
    }
    int64_t outer = 1, dim, inner = 1;
    if (axis == -1) {
        /* mean of everything; the reference broadcasts it to every output element */
        if (Y->elem_count != 1) return SPINN_HIP_EUNSUPPORTED;
        outer = 1;
        dim = X->elem_count;
    } else {
        if (axis < 0 || axis >= ndim) return -1;
        for (int i = 0; i < axis; i++) outer *= X->dims[i];
        dim = X->dims[axis];
        if (merge) {
            for (int i = axis + 1; i < ndim; i++) dim *= X->dims[i];
        } else {
            for (int i = axis + 1; i < ndim; i++) inner *= X->dims[i];
        }
    }
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_reduce_mean(outer, dim, inner, (const float *)X->data, (float *)Y->data, g_spinn_exec.stream);
}

/* Reshape / Flatten / Identity / Unsqueeze: a copy unless the tensors alias
 * (SPINN/run_time/ops/shape/reshape.c:6-14, ops/tensor/flatten.c:3-8,
 * ops/tensor/unsqueeze.c:3-8). */
int op_copy_alias(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 1 || n_out < 1) return -1;
    if (g_spinn_exec.preparing) return 0;
    if (in[0]->data == out[0]->data) return 0;
    size_t bytes = in[0]->size < out[0]->size ? in[0]->size : out[0]->size;
    return spinn_hip_copy(out[0]->data, in[0]->data, bytes, g_spinn_exec.stream);
}

/* ------------------------------------------------------------------------
 * Unfused graph nodes: what graph_opt leaves behind when a Conv cannot absorb
 * the activation or the Add (SPINN/graph_opt.c:301-374), and the tensor ops of
 * detector heads and attention blocks.
 * ---------------------------------------------------------------------- */

/* Add / Sub / Mul / Div with the reference's modulo broadcast
 * (SPINN/run_time/ops/math/add.c:4-21, sub.c:5-20, mul.c:11-63, div.c:5-30). */
static int binary_node(int op, SpinnTensor **in, int n_in, SpinnTensor **out, int n_out) {
    if (n_in < 2 || n_out < 1) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_binary(op, (const float *)in[0]->data, in[0]->elem_count, (const float *)in[1]->data,
                            in[1]->elem_count, (float *)out[0]->data, out[0]->elem_count, g_spinn_exec.stream);
}

int op_add(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return binary_node(SPINN_BINARY_ADD, in, n_in, out, n_out);
}

int op_sub(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return binary_node(SPINN_BINARY_SUB, in, n_in, out, n_out);
}

int op_mul(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return binary_node(SPINN_BINARY_MUL, in, n_in, out, n_out);
}

/* Div / Mod on the dtype of the first input: fp32, int32 or int64, with the
 * reference's modulo broadcast; an empty operand is a no-op
 * (SPINN/run_time/ops/math/div.c:5-52, mod.c:5-50). */
static int typed_binary_node(int op, SpinnTensor **in, int n_in, SpinnTensor **out, int n_out) {
    if (n_in < 2 || n_out < 1) return -1;
    if (in[0]->elem_count == 0 || in[1]->elem_count == 0) return 0;
    const int dt = in[0]->dtype;
    if (dt != ENNF_TYPE_FLOAT32 && dt != ENNF_TYPE_INT32 && dt != ENNF_TYPE_INT64) return SPINN_HIP_EUNSUPPORTED;
    if (in[1]->dtype != dt || out[0]->dtype != dt) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_binary_typed(op, dt, in[0]->data, in[0]->elem_count, in[1]->data, in[1]->elem_count,
                                  out[0]->data, out[0]->elem_count, g_spinn_exec.stream);
}

int op_div(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return typed_binary_node(SPINN_BINARY_DIV, in, n_in, out, n_out);
}

int op_mod(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return typed_binary_node(SPINN_BINARY_MOD, in, n_in, out, n_out);
}

static int unary_node(int op, SpinnTensor **in, int n_in, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    if (out[0]->elem_count < in[0]->elem_count) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_unary(op, (const float *)in[0]->data, (float *)out[0]->data, in[0]->elem_count,
                           g_spinn_exec.stream);
}

/* SPINN/run_time/ops/activation/relu.c:4-16 */
int op_relu(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return unary_node(SPINN_UNARY_RELU, in, n_in, out, n_out);
}

/* SPINN/run_time/ops/activation/sigmoid.c:7-25 */
int op_sigmoid(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    return unary_node(SPINN_UNARY_SIGMOID, in, n_in, out, n_out);
}

/* BatchNormalization, inputs X, scale, B, mean, var; eps from the params,
 * default 1e-5 (SPINN/run_time/ops/norm/batch_norm.c:17-76). */
int op_batch_norm(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 5 || n_out < 1) return -1;
    SpinnTensor *X = in[0];
    if (X->ndim < 2 || out[0]->elem_count < X->elem_count) return -1;
    float eps = 1e-5f;
    if (params && params_size >= sizeof(ENNF_BatchNormParams)) eps = ((const ENNF_BatchNormParams *)params)->epsilon;
    int64_t spatial = 1;
    for (int d = 2; d < X->ndim; d++) spatial *= X->dims[d];
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_batchnorm(X->dims[0], X->dims[1], spatial, (const float *)X->data, (const float *)in[1]->data,
                               (const float *)in[2]->data, (const float *)in[3]->data, (const float *)in[4]->data,
                               eps, (float *)out[0]->data, g_spinn_exec.stream);
}

/* [outer, dim, inner] view of `t` around `axis` (already normalised). */
static void axis_view(const SpinnTensor *t, int axis, int64_t *outer, int64_t *inner) {
    int64_t o = 1, i = 1;
    for (int d = 0; d < axis; d++) o *= t->dims[d];
    for (int d = axis + 1; d < t->ndim; d++) i *= t->dims[d];
    *outer = o;
    *inner = i;
}

/* Softmax along `axis` (default -1) (SPINN/run_time/ops/activation/softmax.c:109-170). */
int op_softmax(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    int axis = -1;
    if (params && params_size >= sizeof(ENNF_AxisParams)) axis = ((const ENNF_AxisParams *)params)->axis;
    const int ndim = in[0]->ndim;
    if (axis < 0) axis += ndim;
    if (axis < 0 || axis >= ndim || out[0]->elem_count < in[0]->elem_count) return -1;
    int64_t outer, inner;
    axis_view(in[0], axis, &outer, &inner);
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_softmax(outer, in[0]->dims[axis], inner, (const float *)in[0]->data, (float *)out[0]->data,
                             g_spinn_exec.stream);
}

/* Concat along `axis` (default 0 without params): each input is one run of
 * dims[axis] * inner floats per outer row (SPINN/run_time/ops/tensor/concat.c:5-26). */
int op_concat(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    int axis = 0;
    if (params && params_size >= sizeof(ENNF_AxisParams)) axis = ((const ENNF_AxisParams *)params)->axis;
    const int ndim = in[0]->ndim;
    if (axis < 0) axis += ndim;
    if (axis < 0 || axis >= ndim) return -1;
    int64_t outer, inner;
    axis_view(in[0], axis, &outer, &inner);
    int64_t row = 0;
    for (int t = 0; t < n_in; t++) {
        if (in[t]->ndim <= axis) return -1;
        row += (int64_t)in[t]->dims[axis] * inner;
    }
    if (outer * row > (int64_t)out[0]->elem_count) return -1;
    if (g_spinn_exec.preparing) return 0;
    SpinnHipBlockCopy blocks[SPINN_HIP_MAX_BLOCKS];
    int64_t off = 0;
    for (int t0 = 0; t0 < n_in; t0 += SPINN_HIP_MAX_BLOCKS) {
        int nb = 0;
        for (int t = t0; t < n_in && nb < SPINN_HIP_MAX_BLOCKS; t++, nb++) {
            const int64_t len = (int64_t)in[t]->dims[axis] * inner;
            blocks[nb] = (SpinnHipBlockCopy){(const float *)in[t]->data, (float *)out[0]->data, len, 0, row, off, len};
            off += len;
        }
        int rc = spinn_hip_block_copy(blocks, nb, outer, g_spinn_exec.stream);
        if (rc) return rc;
    }
    return 0;
}

/* Split along `axis` (default 0); the piece sizes are the outputs' dims[axis]
 * (SPINN/run_time/ops/tensor/split.c:5-26). */
int op_split(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    int axis = 0;
    if (params && params_size >= sizeof(ENNF_SplitParams)) axis = ((const ENNF_SplitParams *)params)->axis;
    const int ndim = in[0]->ndim;
    if (axis < 0) axis += ndim;
    if (axis < 0 || axis >= ndim) return -1;
    int64_t outer, inner;
    axis_view(in[0], axis, &outer, &inner);
    int64_t row = 0;
    for (int t = 0; t < n_out; t++) {
        if (out[t]->ndim <= axis) return -1;
        row += (int64_t)out[t]->dims[axis] * inner;
    }
    if (outer * row > (int64_t)in[0]->elem_count) return -1;
    if (g_spinn_exec.preparing) return 0;
    SpinnHipBlockCopy blocks[SPINN_HIP_MAX_BLOCKS];
    int64_t off = 0;
    for (int t0 = 0; t0 < n_out; t0 += SPINN_HIP_MAX_BLOCKS) {
        int nb = 0;
        for (int t = t0; t < n_out && nb < SPINN_HIP_MAX_BLOCKS; t++, nb++) {
            const int64_t len = (int64_t)out[t]->dims[axis] * inner;
            blocks[nb] = (SpinnHipBlockCopy){(const float *)in[0]->data, (float *)out[t]->data, row, off, len, 0, len};
            off += len;
        }
        int rc = spinn_hip_block_copy(blocks, nb, outer, g_spinn_exec.stream);
        if (rc) return rc;
    }
    return 0;
}

/* Transpose by perm from the params, else reversed dims
 * (SPINN/run_time/ops/shape/transpose.c:14-104). */
int op_transpose(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    if (n_in < 1 || n_out < 1) return -1;
    const int ndim = in[0]->ndim;
    if (ndim < 1 || ndim > ENNF_MAX_DIMS || out[0]->elem_count < in[0]->elem_count) return -1;
    int64_t dims[ENNF_MAX_DIMS];
    int32_t perm[ENNF_MAX_DIMS];
    for (int d = 0; d < ndim; d++) {
        dims[d] = in[0]->dims[d];
        perm[d] = ndim - 1 - d;
    }
    if (params && params_size >= sizeof(ENNF_TransposeParams)) {
        const ENNF_TransposeParams *p = (const ENNF_TransposeParams *)params;
        for (int d = 0; d < ndim; d++) perm[d] = p->perm[d];
    }
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_transpose(ndim, dims, perm, (const float *)in[0]->data, (float *)out[0]->data,
                               g_spinn_exec.stream);
}

/* Resize, nearest only, sizes from the tensors (SPINN/run_time/ops/tensor/resize.c:4-31). */
int op_resize(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 1 || n_out < 1) return -1;
    SpinnTensor *X = in[0], *Y = out[0];
    if (X->ndim != 4 || Y->ndim != 4) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_resize_nearest((int64_t)X->dims[0] * X->dims[1], (int)X->dims[2], (int)X->dims[3],
                                    (int)Y->dims[2], (int)Y->dims[3], (const float *)X->data, (float *)Y->data,
                                    g_spinn_exec.stream);
}

/* ------------------------------------------------------------------------
 * Detector post-processing: the exported YOLOv10 tail after the decoded head
 * (max class score, TopK anchors, gathers, TopK over anchor x class, label and
 * anchor from the flat index).
 * ---------------------------------------------------------------------- */

/* ReduceMax over blocks of |X| / |Y| consecutive elements, whatever the axes
 * parameter says (SPINN/run_time/ops/reduce/reduce_max.c:12-26). */
int op_reduce_max(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 1 || n_out < 1) return -1;
    if (in[0]->dtype != ENNF_TYPE_FLOAT32) return SPINN_HIP_EUNSUPPORTED;
    const uint32_t out_n = out[0]->elem_count;
    if (out_n == 0) return 0;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_reduce_max(out_n, in[0]->elem_count / out_n, (const float *)in[0]->data,
                                (float *)out[0]->data, g_spinn_exec.stream);
}

/* TopK along the last axis, largest first, sorted (SPINN/run_time/ops/tensor/topk.c:20-89).
 * k is the values output's last dimension: the converter's shape inference writes
 * min(K, N) there, the value the reference computes from the K input (:28-59). */
int op_topk(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 2 || n_out < 2) return -1;
    SpinnTensor *X = in[0], *V = out[0], *I = out[1];
    if (X->ndim < 1 || V->ndim != X->ndim || X->dtype != ENNF_TYPE_FLOAT32 || I->dtype != ENNF_TYPE_INT64) return -1;
    const int last = X->ndim - 1;
    const int64_t n = X->dims[last];
    const int64_t k = V->dims[last];
    const int64_t rows = n > 0 ? (int64_t)X->elem_count / n : 0;
    if (k > n || (int64_t)V->elem_count != rows * k || I->elem_count != V->elem_count) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_topk(rows, n, k, (const float *)X->data, (float *)V->data, (int64_t *)I->data,
                          g_spinn_exec.stream);
}

/* GatherElements along `axis` (default 0) (SPINN/run_time/ops/tensor/gather_elements.c:5-76). */
int op_gather_elements(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out,
                       int n_out) {
    if (n_in < 2 || n_out < 1) return -1;
    SpinnTensor *D = in[0], *Ix = in[1], *Y = out[0];
    if (D->dtype != ENNF_TYPE_FLOAT32) return SPINN_HIP_EUNSUPPORTED;
    SpinnHipGatherDesc d;
    memset(&d, 0, sizeof(d));
    d.ndim = D->ndim;
    d.axis = 0;
    if (params && params_size >= sizeof(ENNF_GatherParams)) d.axis = ((const ENNF_GatherParams *)params)->axis;
    if (d.axis < 0) d.axis += d.ndim;
    d.index_dtype = Ix->dtype == ENNF_TYPE_INT64 ? ENNF_TYPE_INT64 : ENNF_TYPE_INT32;
    if (Y->ndim != D->ndim || Ix->elem_count != Y->elem_count) return -1;
    for (int i = 0; i < d.ndim && i < 8; i++) {
        d.in_dims[i] = D->dims[i];
        d.out_dims[i] = Y->dims[i];
    }
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_gather_elements(&d, (const float *)D->data, Ix->data, (float *)Y->data, g_spinn_exec.stream);
}

/* Tile: output coordinate c reads input coordinate c mod dims; the repeats
 * input only shapes the output (SPINN/run_time/ops/tensor/tile.c:6-65). */
int op_tile(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 2 || n_out < 1) return -1;
    SpinnTensor *X = in[0], *Y = out[0];
    if (X->ndim != Y->ndim || X->ndim < 1 || X->ndim > 8) return -1;
    int es = 4; /* element size by dtype, as tile.c:18-24 */
    if (X->dtype == ENNF_TYPE_INT64) es = 8;
    else if (X->dtype == ENNF_TYPE_UINT8 || X->dtype == ENNF_TYPE_INT8) es = 1;
    int64_t id[8], od[8];
    for (int i = 0; i < X->ndim; i++) {
        id[i] = X->dims[i];
        od[i] = Y->dims[i];
    }
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_tile(X->ndim, id, od, es, X->data, Y->data, g_spinn_exec.stream);
}

/* Cast between the tensors' dtypes (SPINN/run_time/ops/tensor/cast.c:13-73). */
int op_cast(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out) {
    (void)params;
    (void)params_size;
    if (n_in < 1 || n_out < 1) return -1;
    if (in[0]->elem_count < out[0]->elem_count) return -1;
    if (g_spinn_exec.preparing) return 0;
    return spinn_hip_cast(in[0]->dtype, out[0]->dtype, out[0]->elem_count, in[0]->data, out[0]->data,
                          g_spinn_exec.stream);
}

/* ------------------------------------------------------------------------
 * Registry and dispatcher (SPINN/run_time/spinn_ops.c:17-228)
 * ---------------------------------------------------------------------- */
static SpinnOpKernel g_op_registry[ENNF_OP_REGISTRY_SIZE];
static int g_registry_ready = 0;

static void registry_init(void) {
    if (g_registry_ready) return;
    g_op_registry[ENNF_OP_Conv] = op_conv2d;
    g_op_registry[ENNF_OP_Gemm] = op_gemm;
    g_op_registry[ENNF_OP_MatMul] = op_matmul;
    g_op_registry[ENNF_OP_MaxPool] = op_maxpool;
    g_op_registry[ENNF_OP_GlobalAveragePool] = op_global_avg_pool;
    g_op_registry[ENNF_OP_ReduceMean] = op_reduce_mean;
    g_op_registry[ENNF_OP_Reshape] = op_copy_alias;
    g_op_registry[ENNF_OP_Flatten] = op_copy_alias;
    g_op_registry[ENNF_OP_Identity] = op_copy_alias;
    g_op_registry[ENNF_OP_Add] = op_add;
    g_op_registry[ENNF_OP_Sub] = op_sub;
    g_op_registry[ENNF_OP_Mul] = op_mul;
    g_op_registry[ENNF_OP_Div] = op_div;
    g_op_registry[ENNF_OP_Relu] = op_relu;
    g_op_registry[ENNF_OP_Sigmoid] = op_sigmoid;
    g_op_registry[ENNF_OP_BatchNormalization] = op_batch_norm;
    g_op_registry[ENNF_OP_Softmax] = op_softmax;
    g_op_registry[ENNF_OP_Concat] = op_concat;
    g_op_registry[ENNF_OP_Split] = op_split;
    g_op_registry[ENNF_OP_Transpose] = op_transpose;
    g_op_registry[ENNF_OP_Resize] = op_resize;
    g_op_registry[ENNF_OP_Mod] = op_mod;
    g_op_registry[ENNF_OP_ReduceMax] = op_reduce_max;
    g_op_registry[ENNF_OP_TopK] = op_topk;
    g_op_registry[ENNF_OP_GatherElements] = op_gather_elements;
    g_op_registry[ENNF_OP_Tile] = op_tile;
    g_op_registry[ENNF_OP_Cast] = op_cast;
    g_op_registry[ENNF_OP_Unsqueeze] = op_copy_alias;
    g_registry_ready = 1;
}

int spinn_dispatch_op(uint16_t op_type, SpinnTensor **inputs, int n_in, void *params, uint16_t params_size,
                      SpinnTensor **outputs, int n_out) {
    registry_init();
    if (op_type >= ENNF_OP_REGISTRY_SIZE) {
        printf("Warning: Op type %d out of range\n", op_type);
        return -1;
    }
    SpinnOpKernel k = g_op_registry[op_type];
    if (!k) {
        if (!g_spinn_exec.preparing) printf("  -> Op %d not implemented (skip)\n", op_type);
        return 0;
    }
    return k(inputs, n_in, params, params_size, outputs, n_out);
}

/* Exposed for tests: is an op id served by a device kernel? */
int spinn_op_registered(uint16_t op_type) {
    registry_init();
    return op_type < ENNF_OP_REGISTRY_SIZE && g_op_registry[op_type] != NULL;
}
