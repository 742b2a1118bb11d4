/*
 * runtime.c - load -> plan -> run over one HBM arena.
 *
 * Load follows the reference's parse of the ENNF file
 * (SPINN/run_time/spinn_runtime.c:21-124): header, graph meta (input/output
 * ids), the tensor meta table placed by tensor id, then the node table with
 * each node's params kept resident; the file stays open for lazy weight reads
 * through the dense entry table at header.reserved[0] (:363-409).
 *
 * Plan (:129-155) runs the static planner, then puts the activation arena in
 * one hipMalloc at the planner's offsets, uploads every weight once into a
 * device weight pool, and runs a prepare pass over the nodes in which each
 * operator re-lays out its weights on the device and reports its scratch
 * need; one workspace of the largest need is then allocated. Nothing is
 * allocated after plan.
 *
 * Run (:298-355) copies input 0 in, launches the nodes in file order on the
 * context's stream (optionally replaying a captured HIP graph), copies output
 * 0 out and waits. Unlike the reference, which ignores operator return codes
 * (:331-345), the first failing node's code is returned.
 */
#include "spinn_host.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define SPINN_PROF_OPS ENNF_OP_REGISTRY_SIZE

/* ---------------- load ---------------- */

static int read_exact(FILE *fp, void *dst, size_t bytes) { return fread(dst, 1, bytes, fp) == bytes ? 0 : -1; }

static void ctx_release(SpinnContext *ctx);

SpinnContext *spinn_load(const char *path) {
    if (!path) return NULL;
    FILE *fp = fopen(path, "rb");
    if (!fp) return NULL;
    SpinnContext *ctx = (SpinnContext *)calloc(1, sizeof(SpinnContext));
    if (!ctx) {
        fclose(fp);
        return NULL;
    }
    ctx->ennf_fp = fp;
    ctx->last_error_node = -1;
    if (read_exact(fp, &ctx->header, sizeof(ENNF_Header))) goto fail;
    if (ctx->header.magic != ENNF_MAGIC) goto fail;
    ctx->flags = ctx->header.flags;
    ctx->num_tensors = ctx->header.num_tensors;
    ctx->num_nodes = ctx->header.num_nodes;
    ctx->num_weights = ctx->header.num_weights;
    ctx->weight_base_offset = ctx->header.weight_data_offset;
    if (ctx->num_tensors == 0 || ctx->num_tensors > 65536) goto fail;
    /* Table sizes the file cannot hold are rejected before anything is sized
     * from them: a node takes at least its 8-byte base record, a tensor its
     * 44-byte meta record. */
    if (fseek(fp, 0, SEEK_END)) goto fail;
    const long file_bytes = ftell(fp);
    if (file_bytes < 0 || (uint64_t)ctx->num_nodes * sizeof(ENNF_NodeBase) > (uint64_t)file_bytes ||
        (uint64_t)ctx->num_tensors * sizeof(ENNF_TensorMeta) > (uint64_t)file_bytes)
        goto fail;

    /* graph meta: u16 n_in, u16 ids[n_in], u16 n_out, u16 ids[n_out] */
    if (fseek(fp, ctx->header.graph_meta_offset, SEEK_SET)) goto fail;
    uint16_t cnt = 0, id = 0;
    if (read_exact(fp, &cnt, 2)) goto fail;
    for (uint16_t i = 0; i < cnt; i++) {
        if (read_exact(fp, &id, 2)) goto fail;
        if (id >= ctx->num_tensors) goto fail;
        if (i < 16) ctx->input_ids[i] = id;
    }
    if (read_exact(fp, &cnt, 2)) goto fail;
    for (uint16_t i = 0; i < cnt; i++) {
        if (read_exact(fp, &id, 2)) goto fail;
        if (id >= ctx->num_tensors) goto fail;
        if (i < 16) ctx->output_ids[i] = id;
    }

    ctx->tensors = (SpinnTensor *)calloc(ctx->num_tensors, sizeof(SpinnTensor));
    if (!ctx->tensors) goto fail;
    if (fseek(fp, ctx->header.tensor_meta_offset, SEEK_SET)) goto fail;
    for (uint32_t i = 0; i < ctx->num_tensors; i++) {
        ENNF_TensorMeta m;
        if (read_exact(fp, &m, sizeof(m))) goto fail;
        if (m.tensor_id >= ctx->num_tensors) goto fail;
        SpinnTensor *t = &ctx->tensors[m.tensor_id];
        /* Every launch and buffer bound is sized from these fields: a tensor
         * whose element count is not the product of its dims, or whose byte
         * size does not fit 32 bits, is a malformed file. */
        if (m.ndim > ENNF_MAX_DIMS) goto fail;
        if (m.ndim > 0) {
            uint64_t prod = 1;
            for (int d = 0; d < m.ndim; d++) {
                prod *= m.dims[d];
                if (prod > UINT32_MAX) goto fail;
            }
            if (prod != m.elem_count) goto fail;
        } else if (m.elem_count > 1) {
            goto fail;
        }
        if ((uint64_t)m.elem_count * ennf_dtype_bytes(m.dtype) > UINT32_MAX) goto fail;
        t->id = m.tensor_id;
        t->dtype = m.dtype;
        t->ndim = m.ndim;
        memcpy(t->dims, m.dims, sizeof(m.dims));
        t->elem_count = m.elem_count;
        t->is_weight = m.is_weight;
        t->ref_count = m.ref_count;
        t->size = (uint32_t)(m.elem_count * ennf_dtype_bytes(m.dtype));
    }

    ctx->nodes = (SpinnNode *)calloc(ctx->num_nodes ? ctx->num_nodes : 1, sizeof(SpinnNode));
    if (!ctx->nodes) goto fail;
    if (fseek(fp, ctx->header.node_table_offset, SEEK_SET)) goto fail;
    for (uint32_t i = 0; i < ctx->num_nodes; i++) {
        ENNF_NodeBase b;
        if (read_exact(fp, &b, sizeof(b))) goto fail;
        SpinnNode *n = &ctx->nodes[i];
        n->op_type = b.op_type;
        n->num_inputs = b.num_inputs > SPINN_MAX_IO ? SPINN_MAX_IO : b.num_inputs;
        n->num_outputs = b.num_outputs > SPINN_MAX_IO ? SPINN_MAX_IO : b.num_outputs;
        n->params_size = b.params_size;
        for (int j = 0; j < b.num_inputs; j++) {
            if (read_exact(fp, &id, 2)) goto fail;
            if (j < SPINN_MAX_IO) n->input_ids[j] = id;
            if (id >= ctx->num_tensors) goto fail;
        }
        for (int j = 0; j < b.num_outputs; j++) {
            if (read_exact(fp, &id, 2)) goto fail;
            if (j < SPINN_MAX_IO) n->output_ids[j] = id;
            if (id >= ctx->num_tensors) goto fail;
        }
        if (b.params_size > 0) {
            n->params = malloc(b.params_size);
            if (!n->params || read_exact(fp, n->params, b.params_size)) goto fail;
        }
    }
    ctx->weight_cache = (void **)calloc(ctx->num_tensors, sizeof(void *));
    if (!ctx->weight_cache) goto fail;
    return ctx;
fail:
    ctx_release(ctx);
    return NULL;
}

/* Host copy of a weight, read lazily from the file and cached
 * (SPINN/run_time/spinn_runtime.c:363-409). */
void *spinn_get_weight(SpinnContext *ctx, uint16_t tensor_id) {
    if (!ctx || tensor_id >= ctx->num_tensors) return NULL;
    if (ctx->weight_cache && ctx->weight_cache[tensor_id]) return ctx->weight_cache[tensor_id];
    SpinnTensor *t = &ctx->tensors[tensor_id];
    if (!t->is_weight || !ctx->ennf_fp) return NULL;
    uint32_t entry_pos = ctx->header.reserved[0] + (uint32_t)tensor_id * (uint32_t)sizeof(ENNF_WeightEntry);
    ENNF_WeightEntry e;
    if (fseek(ctx->ennf_fp, entry_pos, SEEK_SET) || read_exact(ctx->ennf_fp, &e, sizeof(e))) return NULL;
    if (e.data_size == 0) return NULL;
    if (fseek(ctx->ennf_fp, (long)ctx->weight_base_offset + (long)e.data_offset, SEEK_SET)) return NULL;
    void *buf = malloc(e.data_size);
    if (!buf) return NULL;
    if (read_exact(ctx->ennf_fp, buf, e.data_size)) {
        free(buf);
        return NULL;
    }
    if (ctx->weight_cache) ctx->weight_cache[tensor_id] = buf;
    return buf;
}

/* ---------------- plan ---------------- */

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

static int dispatch_node(SpinnContext *ctx, uint32_t i) {
    SpinnNode *node = &ctx->nodes[i];
    if (ctx->node_folded && ctx->node_folded[i]) return 0; /* its consumer reads its input in place */
    SpinnTensor *ins[SPINN_MAX_IO], *outs[SPINN_MAX_IO];
    for (int j = 0; j < node->num_inputs; j++) ins[j] = &ctx->tensors[node->input_ids[j]];
    for (int j = 0; j < node->num_outputs; j++) outs[j] = &ctx->tensors[node->output_ids[j]];
    int transposed = 0;
    if (ctx->node_tsrc)
        for (int s = 0; s < 2 && s < node->num_inputs; s++)
            if (ctx->node_tsrc[2 * i + s] >= 0) {
                ins[s] = &ctx->tensors[ctx->node_tsrc[2 * i + s]];
                transposed |= 1 << s;
            }
    float alpha = 1.f;
    if (ctx->node_tdst && ctx->node_tdst[i] >= 0 && node->num_outputs >= 1) {
        outs[0] = &ctx->tensors[ctx->node_tdst[i]];
        alpha = ctx->node_alpha[i];
    }
    /* A non-empty operand without device memory (a weight whose file entry has
     * no payload, a tensor the planner never placed) would reach a kernel as a
     * null pointer: the node fails instead. */
    for (int j = 0; j < node->num_inputs; j++)
        if (ins[j]->size > 0 && !ins[j]->data) return -1;
    for (int j = 0; j < node->num_outputs; j++)
        if (outs[j]->size > 0 && !outs[j]->data) return -1;
    g_spinn_exec.matmul_alpha = alpha;
    g_spinn_exec.matmul_transposed = transposed;
    int rc = spinn_dispatch_op(node->op_type, ins, node->num_inputs, node->params, node->params_size, outs,
                               node->num_outputs);
    g_spinn_exec.matmul_transposed = 0;
    g_spinn_exec.matmul_alpha = 1.f;
    return rc;
}

/* Reshape, Flatten, Identity and Unsqueeze copy their input unless the two
 * tensors share device bytes (op_copy_alias). The planner (the reference's,
 * whose offsets are kept) gives such an output a region of its own; when no
 * node writes into the input's bytes from this node until the output's last
 * reader, the output reads those bytes in place instead: its device address
 * becomes the input's and the node launches nothing. Graph outputs keep their
 * own region. A node's outputs count as written even when the node is itself
 * an aliased view (conservative: it may only forgo an alias). */
static int view_op(uint16_t op) {
    return op == ENNF_OP_Reshape || op == ENNF_OP_Flatten || op == ENNF_OP_Identity || op == ENNF_OP_Unsqueeze;
}

static int bytes_overlap(const uint8_t *a, uint32_t an, const uint8_t *b, uint32_t bn) {
    return a < b + bn && b < a + an;
}

static void alias_views(SpinnContext *ctx) {
    const uint32_t nt = ctx->num_tensors, nn = ctx->num_nodes;
    int64_t *last = (int64_t *)malloc((size_t)(nt ? nt : 1) * sizeof(int64_t));
    if (!last) return; /* every view keeps its copy */
    for (uint32_t t = 0; t < nt; t++) last[t] = -1;
    for (uint32_t i = 0; i < nn; i++)
        for (int j = 0; j < ctx->nodes[i].num_inputs; j++)
            if (ctx->nodes[i].input_ids[j] < nt) last[ctx->nodes[i].input_ids[j]] = i;
    for (uint32_t o = 0; o < ctx->header.num_outputs && o < 16; o++)
        if (ctx->output_ids[o] < nt) last[ctx->output_ids[o]] = INT64_MAX;
    for (uint32_t k = 0; k < nn; k++) {
        const SpinnNode *nd = &ctx->nodes[k];
        if (!view_op(nd->op_type) || nd->num_inputs < 1 || nd->num_outputs != 1) continue;
        if (nd->input_ids[0] >= nt || nd->output_ids[0] >= nt) continue;
        SpinnTensor *I = &ctx->tensors[nd->input_ids[0]];
        SpinnTensor *O = &ctx->tensors[nd->output_ids[0]];
        if (I->is_weight || O->is_weight || !I->data || !O->data || I->size == 0 || I->size != O->size) continue;
        const int64_t end = last[nd->output_ids[0]];
        if (end == INT64_MAX) continue;
        int ok = 1;
        for (int64_t j = (int64_t)k + 1; j <= end && ok; j++) {
            const SpinnNode *w = &ctx->nodes[j];
            for (int q = 0; q < w->num_outputs && ok; q++) {
                if (w->output_ids[q] >= nt) continue;
                const SpinnTensor *T = &ctx->tensors[w->output_ids[q]];
                if (T->data && T->size && bytes_overlap((const uint8_t *)T->data, T->size, (const uint8_t *)I->data, I->size))
                    ok = 0;
            }
        }
        if (ok) O->data = I->data;
    }
    free(last);
}

/* A Transpose that swaps the last two axes (leading axes in place) and whose
 * only reader is a MatMul operand: the MatMul reads the Transpose's input
 * with the Gemm's transpose flag instead (the tile loaders stage either
 * orientation), provided no node writes into that input's bytes from the
 * Transpose through the MatMul (the MatMul's own output included); the
 * Transpose then launches nothing. Its output tensor is never written. */
static int swaps_last_two(const SpinnNode *nd, int ndim) {
    if (ndim < 2 || ndim > ENNF_MAX_DIMS) return 0;
    int perm[ENNF_MAX_DIMS];
    for (int d = 0; d < ndim; d++) perm[d] = ndim - 1 - d; /* ONNX default: reverse */
    if (nd->params && nd->params_size >= sizeof(ENNF_TransposeParams)) {
        const ENNF_TransposeParams *p = (const ENNF_TransposeParams *)nd->params;
        for (int d = 0; d < ndim; d++) perm[d] = p->perm[d];
    }
    for (int d = 0; d < ndim - 2; d++)
        if (perm[d] != d) return 0;
    return perm[ndim - 2] == ndim - 1 && perm[ndim - 1] == ndim - 2;
}

static int written_between(const SpinnContext *ctx, uint32_t from, uint32_t to, const SpinnTensor *T) {
    for (uint32_t j = from; j <= to; j++) {
        const SpinnNode *w = &ctx->nodes[j];
        if (ctx->node_folded[j]) continue; /* launches nothing */
        for (int q = 0; q < w->num_outputs; q++) {
            if (w->output_ids[q] >= ctx->num_tensors) continue;
            const SpinnTensor *O = &ctx->tensors[w->output_ids[q]];
            if (O->data && O->size && bytes_overlap((const uint8_t *)O->data, O->size, (const uint8_t *)T->data, T->size))
                return 1;
        }
    }
    return 0;
}

static void fold_transposes(SpinnContext *ctx) {
    const uint32_t nt = ctx->num_tensors, nn = ctx->num_nodes;
    free(ctx->node_folded);
    free(ctx->node_tsrc);
    ctx->node_folded = (uint8_t *)calloc(nn ? nn : 1, 1);
    ctx->node_tsrc = (int32_t *)malloc((size_t)(nn ? nn : 1) * 2 * sizeof(int32_t));
    int32_t *producer = (int32_t *)malloc((size_t)(nt ? nt : 1) * sizeof(int32_t));
    uint32_t *readers = (uint32_t *)calloc(nt ? nt : 1, sizeof(uint32_t));
    if (!ctx->node_folded || !ctx->node_tsrc || !producer || !readers) {
        free(ctx->node_folded);
        free(ctx->node_tsrc);
        ctx->node_folded = NULL;
        ctx->node_tsrc = NULL;
        free(producer);
        free(readers);
        return; /* every Transpose runs */
    }
    for (uint32_t i = 0; i < 2 * nn; i++) ctx->node_tsrc[i] = -1;
    for (uint32_t t = 0; t < nt; t++) producer[t] = -1;
    for (uint32_t i = 0; i < nn; i++) {
        const SpinnNode *nd = &ctx->nodes[i];
        for (int q = 0; q < nd->num_outputs; q++)
            if (nd->output_ids[q] < nt) producer[nd->output_ids[q]] = (int32_t)i;
        for (int q = 0; q < nd->num_inputs; q++)
            if (nd->input_ids[q] < nt) readers[nd->input_ids[q]]++;
    }
    for (uint32_t o = 0; o < ctx->header.num_outputs && o < 16; o++)
        if (ctx->output_ids[o] < nt) readers[ctx->output_ids[o]] += 2; /* a graph output is read by the caller */
    for (uint32_t j = 0; j < nn; j++) {
        const SpinnNode *mm = &ctx->nodes[j];
        if (mm->op_type != ENNF_OP_MatMul || mm->num_inputs < 2) continue;
        for (int s = 0; s < 2; s++) {
            const uint16_t x = mm->input_ids[s];
            if (x >= nt || readers[x] != 1 || producer[x] < 0) continue;
            const uint32_t k = (uint32_t)producer[x];
            const SpinnNode *tn = &ctx->nodes[k];
            if (tn->op_type != ENNF_OP_Transpose || tn->num_inputs < 1 || tn->num_outputs != 1) continue;
            if (tn->input_ids[0] >= nt) continue;
            const SpinnTensor *T = &ctx->tensors[tn->input_ids[0]];
            const SpinnTensor *X = &ctx->tensors[x];
            if (!T->data || T->dtype != ENNF_TYPE_FLOAT32 || X->dtype != ENNF_TYPE_FLOAT32 || T->ndim != X->ndim ||
                T->size != X->size || !swaps_last_two(tn, T->ndim))
                continue;
            if (written_between(ctx, k + 1, j, T)) continue;
            ctx->node_folded[k] = 1;
            ctx->node_tsrc[2 * j + s] = (int32_t)tn->input_ids[0];
        }
    }
    free(producer);
    free(readers);
}

/* A Mul of a MatMul's product by a one-element float constant, where the Mul
 * is the product's only reader: the MatMul writes the Mul's output itself with
 * the constant as the Gemm's alpha (alpha * acc is the Mul's own float product,
 * so the bits are the same) and the Mul launches nothing. The MatMul then
 * writes the Mul's output bytes earlier than the plan did: no node from the
 * MatMul until the Mul may read or write them (a tensor the planner placed
 * there and still reads). */
static int touched_between(const SpinnContext *ctx, uint32_t from, uint32_t to, int reads_from, const SpinnTensor *Z) {
    for (uint32_t m = from; m <= to; m++) {
        if (ctx->node_folded[m]) continue;
        const SpinnNode *nd = &ctx->nodes[m];
        if ((int64_t)m >= (int64_t)reads_from) {
            for (int q = 0; q < nd->num_inputs; q++) {
                int32_t id = nd->input_ids[q];
                if (q < 2 && ctx->node_tsrc[2 * m + q] >= 0) id = ctx->node_tsrc[2 * m + q];
                if ((uint32_t)id >= ctx->num_tensors) continue;
                const SpinnTensor *T = &ctx->tensors[id];
                if (T->data && T->size && bytes_overlap((const uint8_t *)T->data, T->size, (const uint8_t *)Z->data, Z->size))
                    return 1;
            }
        }
        if (m == from) continue; /* the MatMul's own output is what moves */
        for (int q = 0; q < nd->num_outputs; q++) {
            if (nd->output_ids[q] >= ctx->num_tensors) continue;
            const SpinnTensor *T = &ctx->tensors[nd->output_ids[q]];
            if (T->data && T->size && bytes_overlap((const uint8_t *)T->data, T->size, (const uint8_t *)Z->data, Z->size))
                return 1;
        }
    }
    return 0;
}

static void fold_scales(SpinnContext *ctx) {
    const uint32_t nt = ctx->num_tensors, nn = ctx->num_nodes;
    free(ctx->node_tdst);
    free(ctx->node_alpha);
    ctx->node_tdst = NULL;
    ctx->node_alpha = NULL;
    if (!ctx->node_folded || !ctx->node_tsrc) return;
    ctx->node_tdst = (int32_t *)malloc((size_t)(nn ? nn : 1) * sizeof(int32_t));
    ctx->node_alpha = (float *)malloc((size_t)(nn ? nn : 1) * sizeof(float));
    int32_t *producer = (int32_t *)malloc((size_t)(nt ? nt : 1) * sizeof(int32_t));
    uint32_t *readers = (uint32_t *)calloc(nt ? nt : 1, sizeof(uint32_t));
    if (!ctx->node_tdst || !ctx->node_alpha || !producer || !readers) {
        free(ctx->node_tdst);
        free(ctx->node_alpha);
        ctx->node_tdst = NULL;
        ctx->node_alpha = NULL;
        free(producer);
        free(readers);
        return; /* every Mul runs */
    }
    for (uint32_t i = 0; i < nn; i++) {
        ctx->node_tdst[i] = -1;
        ctx->node_alpha[i] = 1.f;
    }
    for (uint32_t t = 0; t < nt; t++) producer[t] = -1;
    for (uint32_t i = 0; i < nn; i++) {
        const SpinnNode *nd = &ctx->nodes[i];
        for (int q = 0; q < nd->num_outputs; q++)
            if (nd->output_ids[q] < nt) producer[nd->output_ids[q]] = (int32_t)i;
        for (int q = 0; q < nd->num_inputs; q++)
            if (nd->input_ids[q] < nt) readers[nd->input_ids[q]]++;
    }
    for (uint32_t o = 0; o < ctx->header.num_outputs && o < 16; o++)
        if (ctx->output_ids[o] < nt) readers[ctx->output_ids[o]] += 2;
    for (uint32_t k = 0; k < nn; k++) {
        const SpinnNode *mul = &ctx->nodes[k];
        if (mul->op_type != ENNF_OP_Mul || mul->num_inputs != 2 || mul->num_outputs != 1) continue;
        if (mul->input_ids[0] >= nt || mul->input_ids[1] >= nt || mul->output_ids[0] >= nt) continue;
        for (int s = 0; s < 2; s++) {
            const uint16_t y = mul->input_ids[s], c = mul->input_ids[1 - s];
            const SpinnTensor *Y = &ctx->tensors[y], *S = &ctx->tensors[c], *Z = &ctx->tensors[mul->output_ids[0]];
            if (producer[y] < 0 || readers[y] != 1) continue;
            const uint32_t j = (uint32_t)producer[y];
            const SpinnNode *mm = &ctx->nodes[j];
            if (mm->op_type != ENNF_OP_MatMul || mm->num_outputs != 1 || ctx->node_tdst[j] >= 0) continue;
            if (!S->is_weight || S->dtype != ENNF_TYPE_FLOAT32 || S->elem_count != 1) continue;
            if (Y->dtype != ENNF_TYPE_FLOAT32 || Z->dtype != ENNF_TYPE_FLOAT32 || Z->elem_count != Y->elem_count ||
                !Z->data || !Y->data)
                continue;
            const float *sv = (const float *)spinn_get_weight(ctx, c);
            if (!sv) continue;
            if (touched_between(ctx, j, k - 1, (int)j, Z)) continue;
            ctx->node_tdst[j] = (int32_t)mul->output_ids[0];
            ctx->node_alpha[j] = sv[0];
            ctx->node_folded[k] = 1;
            break;
        }
    }
    free(producer);
    free(readers);
}

/* Bytes of a weight's payload in the file, from its dense entry (0 = none). */
static uint32_t weight_payload_bytes(SpinnContext *ctx, uint16_t tensor_id) {
    uint32_t entry_pos = ctx->header.reserved[0] + (uint32_t)tensor_id * (uint32_t)sizeof(ENNF_WeightEntry);
    ENNF_WeightEntry e;
    if (!ctx->ennf_fp || fseek(ctx->ennf_fp, entry_pos, SEEK_SET) || read_exact(ctx->ennf_fp, &e, sizeof(e)))
        return 0;
    return e.data_size;
}

int spinn_plan(SpinnContext *ctx, uint32_t max_arena_bytes) {
    if (!ctx) return -1;
    /* A weight whose payload is shorter than its tensor would be read past
     * its end by the upload below: reject the file before any device work. */
    for (uint32_t i = 0; i < ctx->num_tensors; i++) {
        SpinnTensor *t = &ctx->tensors[i];
        if (!t->is_weight || t->size == 0) continue;
        uint32_t have = weight_payload_bytes(ctx, (uint16_t)i);
        if (have > 0 && have < t->size) {
            ctx->last_error = -1;
            return -1;
        }
    }
    int peak = spinn_plan_memory(ctx, max_arena_bytes);
    if (peak < 0) return peak;
    if (!ctx->stream && spinn_hip_stream_create(&ctx->stream) != 0) return -2;

    ctx->arena.capacity = (size_t)peak;
    if (peak > 0) {
        void *base = NULL;
        if (spinn_hip_malloc(&base, (size_t)peak) != 0) return -2;
        ctx->arena.base = (uint8_t *)base;
        /* the reference callocs its arena: start from zeros too */
        if (spinn_hip_fill_u32(base, 0u, (size_t)peak, ctx->stream) != 0) return -2; /* peak is a multiple of 16 */
    }
    /* A tensor the planner never placed (neither a model input nor any node's
     * output, in a malformed file) keeps offset 0: it gets device memory only
     * if it fits inside the arena, else none, and a node using it fails. */
    for (uint32_t i = 0; i < ctx->num_tensors; i++) {
        SpinnTensor *t = &ctx->tensors[i];
        if (!t->is_weight && t->size > 0 && (uint64_t)t->offset + t->size <= (uint64_t)peak)
            t->data = ctx->arena.base + t->offset;
    }
    /* SPINN_PLAN_FOLD=0 keeps every view copy and Transpose (each node's output
     * then holds its own bytes, for inspecting intermediate tensors) */
    const char *fold_env = getenv("SPINN_PLAN_FOLD");
    if (fold_env && fold_env[0] == '0') {
        free(ctx->node_folded);
        free(ctx->node_tsrc);
        free(ctx->node_tdst);
        free(ctx->node_alpha);
        ctx->node_folded = NULL;
        ctx->node_tsrc = NULL;
        ctx->node_tdst = NULL;
        ctx->node_alpha = NULL;
    } else {
        alias_views(ctx);
        fold_transposes(ctx);
        fold_scales(ctx);
    }

    /* weights: one device pool, 256-byte aligned entries */
    size_t pool = 0;
    for (uint32_t i = 0; i < ctx->num_tensors; i++) {
        SpinnTensor *t = &ctx->tensors[i];
        if (!t->is_weight) continue;
        if (!spinn_get_weight(ctx, (uint16_t)i)) continue; /* no payload */
        pool = align_up(pool, 256) + t->size;
    }
    if (pool > 0) {
        void *wp = NULL;
        if (spinn_hip_malloc(&wp, pool) != 0) return -2;
        ctx->weight_pool = (uint8_t *)wp;
        ctx->weight_pool_bytes = pool;
        size_t off = 0;
        for (uint32_t i = 0; i < ctx->num_tensors; i++) {
            SpinnTensor *t = &ctx->tensors[i];
            if (!t->is_weight || !ctx->weight_cache[i]) continue;
            off = align_up(off, 256);
            t->data = ctx->weight_pool + off;
            if (spinn_hip_memcpy_h2d(t->data, ctx->weight_cache[i], t->size, ctx->stream) != 0) return -2;
            off += t->size;
        }
    }

    /* prepare pass: weight re-layout and workspace sizing, no compute */
    g_spinn_exec.conv_policy = ctx->conv_policy;
    g_spinn_exec.stream = ctx->stream;
    g_spinn_exec.workspace = NULL;
    g_spinn_exec.workspace_bytes = 0;
    g_spinn_exec.preparing = 1;
    g_spinn_exec.prepare_ws_need = 0;
    int rc = 0;
    for (uint32_t i = 0; i < ctx->num_nodes && rc == 0; i++) {
        int r = dispatch_node(ctx, i);
        if (r < 0) {
            rc = r;
            ctx->last_error = r;
            ctx->last_error_node = (int)i;
        }
    }
    g_spinn_exec.preparing = 0;
    size_t need = g_spinn_exec.prepare_ws_need;
    g_spinn_exec.stream = NULL;
    if (rc == 0 && need > 0) {
        if (spinn_hip_malloc(&ctx->workspace, need) != 0) rc = -2;
        else ctx->workspace_bytes = need;
    }
    /* staging copy of input 0 for resident runs: outside the arena, whose
     * input region later activations reuse */
    SpinnTensor *tin = &ctx->tensors[ctx->input_ids[0]];
    if (rc == 0 && !ctx->input_stage && tin->size > 0 && tin->data) {
        if (spinn_hip_malloc(&ctx->input_stage, tin->size) != 0) rc = -2;
    }
    if (rc == 0 && spinn_hip_stream_sync(ctx->stream) != 0) rc = -2;
    return rc;
}

/* ---------------- profiling ---------------- */

static double g_prof_ms[SPINN_PROF_OPS];
static uint64_t g_prof_calls[SPINN_PROF_OPS];
static int g_prof_enabled = -1;

static void prof_init_once(void) {
    if (g_prof_enabled >= 0) return;
    const char *e = getenv("SPINN_PROFILE");
    g_prof_enabled = (e && e[0] != '0') ? 1 : 0;
}

typedef struct {
    void **events; /* num_nodes + 1 */
    float *node_ms;
    uint32_t n;
} ProfState;

static ProfState *prof_state(SpinnContext *ctx) {
    if (ctx->prof_state) return (ProfState *)ctx->prof_state;
    ProfState *ps = (ProfState *)calloc(1, sizeof(ProfState));
    if (!ps) return NULL;
    ps->n = ctx->num_nodes;
    ps->events = (void **)calloc(ps->n + 1, sizeof(void *));
    ps->node_ms = (float *)calloc(ps->n ? ps->n : 1, sizeof(float));
    if (!ps->events || !ps->node_ms) {
        free(ps->events);
        free(ps->node_ms);
        free(ps);
        return NULL;
    }
    for (uint32_t i = 0; i <= ps->n; i++) {
        if (spinn_hip_event_create(&ps->events[i]) != 0) ps->events[i] = NULL;
    }
    ctx->prof_state = ps;
    return ps;
}

static void prof_free(SpinnContext *ctx) {
    ProfState *ps = (ProfState *)ctx->prof_state;
    if (!ps) return;
    for (uint32_t i = 0; i <= ps->n; i++) spinn_hip_event_destroy(ps->events[i]);
    free(ps->events);
    free(ps->node_ms);
    free(ps);
    ctx->prof_state = NULL;
}

/* Top-12 op types by accumulated device time (SPINN/run_time/spinn_runtime.c:269-296). */
void spinn_set_profiling(int on) { g_prof_enabled = on ? 1 : 0; }

void spinn_profile_dump(void) {
    if (g_prof_enabled <= 0) return;
    double total = 0;
    for (int i = 0; i < SPINN_PROF_OPS; i++) total += g_prof_ms[i];
    if (total <= 0) return;
    fprintf(stderr, "\n===== SPINN per-op profile (device time) =====\n");
    fprintf(stderr, "%-6s %10s %10s %8s %8s\n", "op_id", "calls", "total_ms", "ms/call", "%total");
    int used[SPINN_PROF_OPS] = {0};
    for (int r = 0; r < 12; r++) {
        int best = -1;
        for (int i = 0; i < SPINN_PROF_OPS; i++)
            if (!used[i] && g_prof_ms[i] > 0 && (best < 0 || g_prof_ms[i] > g_prof_ms[best])) best = i;
        if (best < 0) break;
        used[best] = 1;
        fprintf(stderr, "%-6d %10lu %10.3f %8.4f %7.1f%%\n", best, (unsigned long)g_prof_calls[best], g_prof_ms[best],
                g_prof_ms[best] / (double)g_prof_calls[best], 100.0 * g_prof_ms[best] / total);
    }
    fprintf(stderr, "Total tracked: %.3f ms\n", total);
}

int spinn_node_times(SpinnContext *ctx, float *ms_out, int max_nodes) {
    if (!ctx || !ms_out || !ctx->prof_state) return 0;
    ProfState *ps = (ProfState *)ctx->prof_state;
    int n = (int)ps->n < max_nodes ? (int)ps->n : max_nodes;
    memcpy(ms_out, ps->node_ms, (size_t)n * sizeof(float));
    return n;
}

/* ---------------- run ---------------- */

static int run_nodes(SpinnContext *ctx, ProfState *ps) {
    int first = 0;
    for (uint32_t i = 0; i < ctx->num_nodes; i++) {
        if (ps && ps->events[i]) spinn_hip_event_record(ps->events[i], ctx->stream);
        int r = dispatch_node(ctx, i);
        if (r < 0 && first == 0) {
            first = r;
            ctx->last_error = r;
            ctx->last_error_node = (int)i;
        }
    }
    if (ps && ps->events[ctx->num_nodes]) spinn_hip_event_record(ps->events[ctx->num_nodes], ctx->stream);
    return first;
}

static int run_impl(SpinnContext *ctx, void *input_data, void *output_data, int restore_stage) {
    if (!ctx || !ctx->stream) return -1;
    prof_init_once();
    ctx->last_error = 0;
    ctx->last_error_node = -1;
    int rc = 0;
    SpinnTensor *tin = &ctx->tensors[ctx->input_ids[0]];
    if (input_data && tin->data) {
        rc = spinn_hip_memcpy_h2d(tin->data, input_data, tin->size, ctx->stream);
        if (rc) return rc;
    } else if (restore_stage && tin->data) {
        /* ordered on the stream before the node loop (eager or graph replay) */
        rc = spinn_hip_copy(tin->data, ctx->input_stage, tin->size, ctx->stream);
        if (rc) return rc;
    }
    g_spinn_exec.conv_policy = ctx->conv_policy;
    g_spinn_exec.stream = ctx->stream;
    g_spinn_exec.workspace = ctx->workspace;
    g_spinn_exec.workspace_bytes = ctx->workspace_bytes;
    ProfState *ps = g_prof_enabled ? prof_state(ctx) : NULL;
    if (ctx->use_graph && !ps) {
        if (!ctx->graph_exec) {
            rc = spinn_hip_graph_capture_begin(ctx->stream);
            if (rc == 0) {
                int r = run_nodes(ctx, NULL);
                void *exec = NULL;
                int e = spinn_hip_graph_capture_end(ctx->stream, &exec);
                /* A node that failed left its launches out of the capture: keep
                 * no graph, so the next run captures again and fails again
                 * instead of replaying the incomplete one. */
                if (r == 0 && e == 0) ctx->graph_exec = exec;
                else if (exec) spinn_hip_graph_destroy(exec);
                rc = r ? r : e;
            }
        }
        if (rc == 0) rc = spinn_hip_graph_launch(ctx->graph_exec, ctx->stream);
    } else {
        rc = run_nodes(ctx, ps);
    }
    g_spinn_exec.stream = NULL;
    g_spinn_exec.workspace = NULL;
    g_spinn_exec.workspace_bytes = 0;
    SpinnTensor *tout = &ctx->tensors[ctx->output_ids[0]];
    if (rc == 0 && output_data && tout->data) rc = spinn_hip_memcpy_d2h(output_data, tout->data, tout->size, ctx->stream);
    int s = spinn_hip_stream_sync(ctx->stream);
    if (rc == 0) rc = s;
    if (rc == 0) rc = spinn_hip_device_status(); /* a kernel that could not finish its work */
    if (ps && rc == 0) {
        for (uint32_t i = 0; i < ctx->num_nodes; i++) {
            float ms = 0.f;
            if (ps->events[i] && ps->events[i + 1] &&
                spinn_hip_event_elapsed_ms(ps->events[i], ps->events[i + 1], &ms) == 0) {
                ps->node_ms[i] = ms;
                uint16_t op = ctx->nodes[i].op_type;
                if (op < SPINN_PROF_OPS) {
                    g_prof_ms[op] += ms;
                    g_prof_calls[op] += 1;
                }
            }
        }
    }
    return rc;
}

int spinn_run(SpinnContext *ctx, void *input_data, void *output_data) {
    return run_impl(ctx, input_data, output_data, 0);
}

int spinn_run_resident(SpinnContext *ctx) {
    if (!ctx || !ctx->input_stage || !ctx->input_staged) return -1;
    return run_impl(ctx, NULL, NULL, 1);
}

int spinn_stage_input(SpinnContext *ctx, const void *host, size_t bytes) {
    if (!ctx || !ctx->input_stage) return -1;
    SpinnTensor *tin = &ctx->tensors[ctx->input_ids[0]];
    if (host) {
        if (bytes != tin->size) return -1;
        int rc = spinn_hip_memcpy_h2d(ctx->input_stage, host, bytes, ctx->stream);
        if (rc == 0) rc = spinn_hip_stream_sync(ctx->stream);
        if (rc) return rc;
    } else if (bytes != 0) {
        return -1;
    }
    ctx->input_staged = 1;
    return 0;
}

void *spinn_input_stage_ptr(SpinnContext *ctx) { return ctx ? ctx->input_stage : NULL; }

int spinn_set_graph_mode(SpinnContext *ctx, int enable) {
    if (!ctx) return -1;
    if (!enable && ctx->graph_exec) {
        spinn_hip_graph_destroy(ctx->graph_exec);
        ctx->graph_exec = NULL;
    }
    ctx->use_graph = enable ? 1 : 0;
    return 0;
}

int spinn_set_conv_policy(SpinnContext *ctx, int policy) {
    if (!ctx || ctx->arena.base || ctx->weight_pool) return -1;
    if (policy < SPINN_CONV_POLICY_AUTO || policy > SPINN_CONV_POLICY_WINOGRAD) return -1;
    ctx->conv_policy = policy;
    return 0;
}

int spinn_tensor_upload(SpinnContext *ctx, uint16_t tensor_id, const void *host, size_t bytes) {
    if (!ctx || tensor_id >= ctx->num_tensors || !host) return -1;
    SpinnTensor *t = &ctx->tensors[tensor_id];
    if (!t->data || bytes > t->size) return -1;
    int rc = spinn_hip_memcpy_h2d(t->data, host, bytes, ctx->stream);
    if (rc == 0) rc = spinn_hip_stream_sync(ctx->stream);
    return rc;
}

int spinn_tensor_download(SpinnContext *ctx, uint16_t tensor_id, void *host, size_t bytes) {
    if (!ctx || tensor_id >= ctx->num_tensors || !host) return -1;
    SpinnTensor *t = &ctx->tensors[tensor_id];
    if (!t->data || bytes > t->size) return -1;
    int rc = spinn_hip_memcpy_d2h(host, t->data, bytes, ctx->stream);
    if (rc == 0) rc = spinn_hip_stream_sync(ctx->stream);
    return rc;
}

/* ---------------- free ---------------- */

void spinn_free_packed(SpinnContext *ctx) {
    if (!ctx || !ctx->tensors) return;
    for (uint32_t i = 0; i < ctx->num_tensors; i++) {
        if (ctx->tensors[i].packed_data) spinn_packed_release(ctx->tensors[i].packed_data);
        ctx->tensors[i].packed_data = NULL;
    }
}

static void ctx_release(SpinnContext *ctx) {
    if (!ctx) return;
    if (ctx->stream) spinn_hip_stream_sync(ctx->stream);
    prof_free(ctx);
    if (ctx->graph_exec) spinn_hip_graph_destroy(ctx->graph_exec);
    spinn_free_packed(ctx);
    if (ctx->workspace) spinn_hip_free(ctx->workspace);
    if (ctx->input_stage) spinn_hip_free(ctx->input_stage);
    if (ctx->weight_pool) spinn_hip_free(ctx->weight_pool);
    if (ctx->arena.base) spinn_hip_free(ctx->arena.base);
    if (ctx->stream) spinn_hip_stream_destroy(ctx->stream);
    if (ctx->weight_cache) {
        for (uint32_t i = 0; i < ctx->num_tensors; i++) free(ctx->weight_cache[i]);
        free(ctx->weight_cache);
    }
    if (ctx->nodes) {
        for (uint32_t i = 0; i < ctx->num_nodes; i++) free(ctx->nodes[i].params);
        free(ctx->nodes);
    }
    free(ctx->node_folded);
    free(ctx->node_tsrc);
    free(ctx->node_tdst);
    free(ctx->node_alpha);
    free(ctx->tensors);
    if (ctx->ennf_fp) fclose(ctx->ennf_fp);
    free(ctx);
}

void spinn_free(SpinnContext *ctx) { ctx_release(ctx); }
