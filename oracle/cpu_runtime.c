/*
 * cpu_runtime.c - ORACLE (test infrastructure only): runs an ENNF model on the
 * CPU with the restated operators of spinn_cpu.c.
 *
 * Loading follows SPINN/run_time/spinn_runtime.c:21-124 (header, graph meta,
 * tensor meta by id, node table, weights through the dense entry table at
 * header.reserved[0]); every activation gets its own buffer so intermediates
 * stay readable after a run (per-layer parity checks); nodes run in file
 * order as in SPINN/run_time/spinn_runtime.c:309-346, with the operand
 * conventions of the reference operators.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../include/ennf_format.h"
#include "oracle.h"

typedef struct {
    uint8_t dtype, ndim, is_weight;
    uint32_t dims[ENNF_MAX_DIMS];
    uint32_t elems, bytes;
    void *data;
} OT;

typedef struct {
    uint16_t op;
    uint8_t nin, nout;
    uint16_t in[16], out[16];
    uint16_t psize;
    uint8_t *params;
} ON;

struct OracleModel {
    ENNF_Header h;
    uint16_t in_ids[16], out_ids[16];
    uint32_t nt, nn;
    OT *t;
    ON *n;
    int winograd;
};

static int rd(FILE *f, void *p, size_t b) { return fread(p, 1, b, f) == b ? 0 : -1; }

void oracle_model_free(OracleModel *m) {
    if (!m) return;
    if (m->t) for (uint32_t i = 0; i < m->nt; i++) free(m->t[i].data);
    if (m->n) for (uint32_t i = 0; i < m->nn; i++) free(m->n[i].params);
    free(m->t);
    free(m->n);
    free(m);
}

OracleModel *oracle_model_load(const char *path) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    OracleModel *m = (OracleModel *)calloc(1, sizeof(*m));
    uint16_t cnt, id;
    if (!m || rd(f, &m->h, sizeof(m->h)) || m->h.magic != ENNF_MAGIC) goto fail;
    m->nt = m->h.num_tensors;
    m->nn = m->h.num_nodes;
    if (fseek(f, m->h.graph_meta_offset, SEEK_SET) || rd(f, &cnt, 2)) goto fail;
    for (int i = 0; i < cnt; i++) { if (rd(f, &id, 2)) goto fail; if (i < 16) m->in_ids[i] = id; }
    if (rd(f, &cnt, 2)) goto fail;
    for (int i = 0; i < cnt; i++) { if (rd(f, &id, 2)) goto fail; if (i < 16) m->out_ids[i] = id; }
    m->t = (OT *)calloc(m->nt, sizeof(OT));
    m->n = (ON *)calloc(m->nn ? m->nn : 1, sizeof(ON));
    if (!m->t || !m->n) goto fail;
    if (fseek(f, m->h.tensor_meta_offset, SEEK_SET)) goto fail;
    for (uint32_t i = 0; i < m->nt; i++) {
        ENNF_TensorMeta tm;
        if (rd(f, &tm, sizeof(tm)) || tm.tensor_id >= m->nt) goto fail;
        OT *t = &m->t[tm.tensor_id];
        t->dtype = tm.dtype;
        t->ndim = tm.ndim;
        memcpy(t->dims, tm.dims, sizeof(t->dims));
        t->elems = tm.elem_count;
        t->is_weight = tm.is_weight;
        t->bytes = (uint32_t)(tm.elem_count * ennf_dtype_bytes(tm.dtype));
    }
    if (fseek(f, m->h.node_table_offset, SEEK_SET)) goto fail;
    for (uint32_t i = 0; i < m->nn; i++) {
        ENNF_NodeBase b;
        if (rd(f, &b, sizeof(b)) || b.num_inputs > 16 || b.num_outputs > 16) goto fail;
        ON *n = &m->n[i];
        n->op = b.op_type;
        n->nin = b.num_inputs;
        n->nout = b.num_outputs;
        n->psize = b.params_size;
        if (rd(f, n->in, 2u * b.num_inputs) || rd(f, n->out, 2u * b.num_outputs)) goto fail;
        if (b.params_size) {
            n->params = (uint8_t *)malloc(b.params_size);
            if (!n->params || rd(f, n->params, b.params_size)) goto fail;
        }
    }
    for (uint32_t i = 0; i < m->nt; i++) {
        OT *t = &m->t[i];
        if (t->is_weight) {
            ENNF_WeightEntry e;
            if (fseek(f, m->h.reserved[0] + i * sizeof(ENNF_WeightEntry), SEEK_SET) || rd(f, &e, sizeof(e))) goto fail;
            if (e.data_size == 0) continue;
            t->data = malloc(e.data_size);
            if (!t->data || fseek(f, (long)m->h.weight_data_offset + e.data_offset, SEEK_SET) ||
                rd(f, t->data, e.data_size))
                goto fail;
        } else if (t->bytes) {
            t->data = calloc(1, t->bytes);
            if (!t->data) goto fail;
        }
    }
    fclose(f);
    return m;
fail:
    fclose(f);
    oracle_model_free(m);
    return NULL;
}

int oracle_model_num_nodes(const OracleModel *m) { return m ? (int)m->nn : 0; }

void oracle_model_set_winograd(OracleModel *m, int on) {
    if (m) m->winograd = on;
}

long oracle_model_tensor(const OracleModel *m, int id, void *dst, size_t bytes) {
    if (!m || id < 0 || (uint32_t)id >= m->nt || !m->t[id].data) return -1;
    size_t b = m->t[id].bytes < bytes ? m->t[id].bytes : bytes;
    memcpy(dst, m->t[id].data, b);
    return (long)b;
}

/* conv node: operand conventions of SPINN/run_time/ops/conv/conv2d.c:96-145 */
static int run_conv(OracleModel *m, ON *n) {
    const ENNF_ConvParams *p = n->psize >= sizeof(ENNF_ConvParams) ? (const ENNF_ConvParams *)n->params : NULL;
    const int act = p ? p->reserved : 0;
    const int has_res = act == 4 || act == 5;
    const int nreal = has_res ? n->nin - 1 : n->nin;
    OT *X = &m->t[n->in[0]], *W = &m->t[n->in[1]], *Y = &m->t[n->out[0]];
    OracleConv c;
    c.n = X->dims[0]; c.c = X->dims[1]; c.h = X->dims[2]; c.w = X->dims[3];
    c.oc = W->dims[0]; c.kh = W->dims[2]; c.kw = W->dims[3];
    c.oh = Y->dims[2]; c.ow = Y->dims[3];
    c.sh = c.sw = 1; c.ph = c.pw = 0; c.group = 1; c.act = act;
    if (p) {
        if (p->group > 0) c.group = p->group;
        if (p->kernel_shape[0] > 0) c.kh = p->kernel_shape[0];
        if (p->kernel_shape[1] > 0) c.kw = p->kernel_shape[1];
        if (p->strides[0] > 0) c.sh = p->strides[0];
        if (p->strides[1] > 0) c.sw = p->strides[1];
        c.ph = p->pads[0];
        c.pw = p->pads[1];
        if (p->auto_pad == 1 || p->auto_pad == 2) {
            int ph = (c.oh - 1) * c.sh + c.kh - c.h, pw = (c.ow - 1) * c.sw + c.kw - c.w;
            if (ph < 0) ph = 0;
            if (pw < 0) pw = 0;
            c.ph = p->auto_pad == 1 ? ph / 2 : (ph + 1) / 2;
            c.pw = p->auto_pad == 1 ? pw / 2 : (pw + 1) / 2;
        }
    }
    const float *bias = (nreal > 2 && m->t[n->in[2]].data) ? (const float *)m->t[n->in[2]].data : NULL;
    const float *R = has_res ? (const float *)m->t[n->in[n->nin - 1]].data : NULL;
    if (m->winograd && c.kh == 3 && c.kw == 3 && c.sh == 1 && c.sw == 1 && c.group == 1)
        return oracle_winograd(&c, (const float *)X->data, (const float *)W->data, bias, R, (float *)Y->data);
    return oracle_conv2d(&c, (const float *)X->data, (const float *)W->data, bias, R, (float *)Y->data);
}

static int run_node(OracleModel *m, ON *n) {
    OT *X = &m->t[n->in[0]], *Y = &m->t[n->out[0]];
    switch (n->op) {
    case ENNF_OP_Conv:
        return run_conv(m, n);
    case ENNF_OP_Gemm: {
        const ENNF_GemmParams *p = n->psize >= sizeof(ENNF_GemmParams) ? (const ENNF_GemmParams *)n->params : NULL;
        const int ta = p ? p->transA : 0, tb = p ? p->transB : 0;
        const float alpha = p ? p->alpha : 1.0f, beta = p ? p->beta : 1.0f;
        OT *B = &m->t[n->in[1]];
        OT *Cb = (n->nin > 2 && m->t[n->in[2]].data) ? &m->t[n->in[2]] : NULL;
        const int M = ta ? X->dims[1] : X->dims[0], K = ta ? X->dims[0] : X->dims[1];
        const int N = tb ? B->dims[0] : B->dims[1];
        return oracle_gemm(M, N, K, ta, tb, alpha, beta, (const float *)X->data, (const float *)B->data,
                           Cb ? (const float *)Cb->data : NULL, Cb ? (int)Cb->elems : 0, (float *)Y->data);
    }
    case ENNF_OP_MatMul: {
        OT *B = &m->t[n->in[1]];
        const int an = X->ndim, bn = B->ndim;
        const int M = X->dims[an - 2], K = X->dims[an - 1], N = B->dims[bn - 1];
        int batch = 1, bb = 1;
        for (int i = 0; i < an - 2; i++) batch *= X->dims[i];
        for (int i = 0; i < bn - 2; i++) bb *= B->dims[i];
        if ((int)B->dims[bn - 2] != K || batch != bb) return -1;
        return oracle_matmul(batch, M, N, K, (const float *)X->data, (const float *)B->data, (float *)Y->data);
    }
    case ENNF_OP_MaxPool: {
        const ENNF_PoolParams *p = n->psize >= sizeof(ENNF_PoolParams) ? (const ENNF_PoolParams *)n->params : NULL;
        int kh = 1, kw = 1, sh = 1, sw = 1, ph = 0, pw = 0;
        if (p) { kh = p->kernel_shape[0]; kw = p->kernel_shape[1]; sh = p->strides[0]; sw = p->strides[1];
                 ph = p->pads[0]; pw = p->pads[1]; }
        oracle_maxpool(X->dims[0], X->dims[1], X->dims[2], X->dims[3], Y->dims[2], Y->dims[3], kh, kw, sh, sw, ph, pw,
                       (const float *)X->data, (float *)Y->data);
        return 0;
    }
    case ENNF_OP_GlobalAveragePool:
        oracle_reduce_mean((long)X->dims[0] * X->dims[1], (long)X->dims[2] * X->dims[3], 1, (const float *)X->data,
                           (float *)Y->data);
        return 0;
    case ENNF_OP_ReduceMean: {
        /* axes given explicitly by the models this runner serves: mean over
         * axes[0].. with trailing axes merged (reduce_mean.c:14-21,62-75) */
        const ENNF_ReduceParams *p = n->psize >= sizeof(ENNF_ReduceParams) ? (const ENNF_ReduceParams *)n->params : NULL;
        if (!p || p->num_axes == 0) return -1;
        int axis = p->axes[0];
        if (axis < 0) axis += X->ndim;
        const int merge = p->num_axes > 1 && axis + p->num_axes == X->ndim;
        long outer = 1, dim = X->dims[axis], inner = 1;
        for (int i = 0; i < axis; i++) outer *= X->dims[i];
        for (int i = axis + 1; i < X->ndim; i++) {
            if (merge) dim *= X->dims[i];
            else inner *= X->dims[i];
        }
        oracle_reduce_mean(outer, dim, inner, (const float *)X->data, (float *)Y->data);
        return 0;
    }
    case ENNF_OP_Reshape:
    case ENNF_OP_Flatten:
    case ENNF_OP_Identity:
        memcpy(Y->data, X->data, X->bytes < Y->bytes ? X->bytes : Y->bytes);
        return 0;
    case ENNF_OP_Add:
    case ENNF_OP_Sub:
    case ENNF_OP_Mul:
    case ENNF_OP_Div: {
        OT *B = &m->t[n->in[1]];
        if (n->nin < 2 || X->elems == 0 || B->elems == 0) return n->nin < 2 ? -1 : 0;
        if (n->op == ENNF_OP_Div && X->dtype != ENNF_TYPE_FLOAT32)
            return oracle_binary_typed(3, X->dtype, X->data, X->elems, B->data, B->elems, Y->data, Y->elems);
        const int op = n->op == ENNF_OP_Add ? 0 : n->op == ENNF_OP_Sub ? 1 : n->op == ENNF_OP_Mul ? 2 : 3;
        oracle_binary(op, (const float *)X->data, X->elems, (const float *)B->data, B->elems, (float *)Y->data,
                      Y->elems);
        return 0;
    }
    case ENNF_OP_Relu:
    case ENNF_OP_Sigmoid:
        oracle_unary(n->op == ENNF_OP_Relu ? 0 : 1, (const float *)X->data, (float *)Y->data, X->elems);
        return 0;
    case ENNF_OP_BatchNormalization: {
        if (n->nin < 5) return -1;
        const ENNF_BatchNormParams *p =
            n->psize >= sizeof(ENNF_BatchNormParams) ? (const ENNF_BatchNormParams *)n->params : NULL;
        long spatial = 1;
        for (int d = 2; d < X->ndim; d++) spatial *= X->dims[d];
        oracle_batchnorm(X->dims[0], X->dims[1], spatial, (const float *)X->data,
                         (const float *)m->t[n->in[1]].data, (const float *)m->t[n->in[2]].data,
                         (const float *)m->t[n->in[3]].data, (const float *)m->t[n->in[4]].data,
                         p ? p->epsilon : 1e-5f, (float *)Y->data);
        return 0;
    }
    case ENNF_OP_Softmax:
    case ENNF_OP_Concat:
    case ENNF_OP_Split: {
        /* axis defaults: Softmax -1, Concat / Split 0 (softmax.c:113, concat.c:7, split.c:7) */
        int axis = n->op == ENNF_OP_Softmax ? -1 : 0;
        if (n->psize >= 4) memcpy(&axis, n->params, 4);
        if (axis < 0) axis += X->ndim;
        if (axis < 0 || axis >= X->ndim) return -1;
        long outer = 1, inner = 1;
        for (int d = 0; d < axis; d++) outer *= X->dims[d];
        for (int d = axis + 1; d < X->ndim; d++) inner *= X->dims[d];
        if (n->op == ENNF_OP_Softmax) {
            oracle_softmax(outer, X->dims[axis], inner, (const float *)X->data, (float *)Y->data);
        } else if (n->op == ENNF_OP_Concat) {
            const float *xs[16];
            long sizes[16];
            for (int t = 0; t < n->nin; t++) {
                xs[t] = (const float *)m->t[n->in[t]].data;
                sizes[t] = m->t[n->in[t]].dims[axis];
            }
            oracle_concat(n->nin, xs, sizes, outer, inner, (float *)Y->data);
        } else {
            float *ys[16];
            long sizes[16];
            for (int t = 0; t < n->nout; t++) {
                ys[t] = (float *)m->t[n->out[t]].data;
                sizes[t] = m->t[n->out[t]].dims[axis];
            }
            oracle_split(n->nout, ys, sizes, outer, inner, (const float *)X->data);
        }
        return 0;
    }
    case ENNF_OP_Transpose: {
        long dims[8];
        int perm[8];
        for (int d = 0; d < X->ndim; d++) {
            dims[d] = X->dims[d];
            perm[d] = X->ndim - 1 - d;
        }
        if (n->psize >= sizeof(ENNF_TransposeParams))
            for (int d = 0; d < X->ndim; d++) perm[d] = ((const ENNF_TransposeParams *)n->params)->perm[d];
        oracle_transpose(X->ndim, dims, perm, (const float *)X->data, (float *)Y->data);
        return 0;
    }
    case ENNF_OP_Mod: {
        OT *B = &m->t[n->in[1]];
        if (n->nin < 2) return -1;
        return oracle_binary_typed(4, X->dtype, X->data, X->elems, B->data, B->elems, Y->data, Y->elems);
    }
    case ENNF_OP_Unsqueeze:
        memcpy(Y->data, X->data, X->bytes < Y->bytes ? X->bytes : Y->bytes);
        return 0;
    case ENNF_OP_ReduceMax:
        if (Y->elems == 0) return 0;
        oracle_reduce_max(Y->elems, X->elems / Y->elems, (const float *)X->data, (float *)Y->data);
        return 0;
    case ENNF_OP_TopK: {
        /* K from the second input, rows over the last axis (topk.c:28-56) */
        if (n->nin < 2 || n->nout < 2) return -1;
        const int64_t kv = *(const int64_t *)m->t[n->in[1]].data;
        const long last = X->dims[X->ndim - 1];
        const long rows = last ? (long)X->elems / last : 0;
        return oracle_topk(rows, last, kv, (const float *)X->data, (float *)Y->data,
                           (int64_t *)m->t[n->out[1]].data);
    }
    case ENNF_OP_GatherElements: {
        int axis = 0;
        if (n->psize >= sizeof(ENNF_GatherParams)) axis = ((const ENNF_GatherParams *)n->params)->axis;
        if (axis < 0) axis += X->ndim;
        OT *I = &m->t[n->in[1]];
        oracle_gather_elements(X->ndim, X->dims, Y->dims, axis, (const float *)X->data, I->data, I->dtype,
                               (float *)Y->data, Y->elems);
        return 0;
    }
    case ENNF_OP_Tile: {
        const int es = X->dtype == ENNF_TYPE_INT64 ? 8 : (X->dtype == ENNF_TYPE_UINT8 || X->dtype == ENNF_TYPE_INT8) ? 1 : 4;
        oracle_tile(X->ndim, X->dims, Y->dims, es, X->data, Y->data);
        return 0;
    }
    case ENNF_OP_Cast:
        return oracle_cast(X->dtype, Y->dtype, Y->elems, X->data, Y->data);
    case ENNF_OP_Resize:
        if (X->ndim != 4 || Y->ndim != 4) return -1;
        oracle_resize_nearest((long)X->dims[0] * X->dims[1], X->dims[2], X->dims[3], Y->dims[2], Y->dims[3],
                              (const float *)X->data, (float *)Y->data);
        return 0;
    default:
        fprintf(stderr, "oracle: op %d not implemented\n", n->op);
        return -2;
    }
}

int oracle_model_run(OracleModel *m, const float *input, float *output) {
    if (!m) return -1;
    OT *ti = &m->t[m->in_ids[0]];
    if (input && ti->data) memcpy(ti->data, input, ti->bytes);
    for (uint32_t i = 0; i < m->nn; i++) {
        int r = run_node(m, &m->n[i]);
        if (r) return r;
    }
    OT *to = &m->t[m->out_ids[0]];
    if (output && to->data) memcpy(output, to->data, to->bytes);
    return 0;
}
