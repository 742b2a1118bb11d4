/*
 * planner.c - static activation-arena planner.
 *
 * Restates the reference planner's algorithm so that offsets, and therefore
 * the HBM arena layout, are identical to the reference's host arena
 * (SPINN/run_time/spinn_memory_planner.c:146-252):
 *   - free space is a list of [offset, size) blocks kept in offset order,
 *     initially one block [0, max_arena_bytes or 0xFFFFFFFF);
 *   - requests are rounded up to 16 bytes and served best-fit: the smallest
 *     block that fits, the lowest offset among equal sizes; an exact fit
 *     consumes the block, otherwise the block's front is split off (:56-98);
 *   - a release re-inserts the block in order and merges it with its
 *     successor, then with its predecessor (:103-141);
 *   - model inputs are placed first (:171-192); then per node in file order
 *     the outputs are placed, after which every activation input whose
 *     remaining reference count reaches zero is released, model outputs
 *     excepted (:195-241);
 *   - the return value is the largest block end ever handed out (clamped to
 *     INT_MAX), or SPINN_MEM_ERR_NOMEM when a request does not fit.
 * The list lives in a growable array instead of malloc'd nodes.
 */
#include "spinn_host.h"
#include <stdlib.h>
#include <string.h>

typedef struct {
    uint32_t offset;
    uint32_t size;
} FreeBlock;

typedef struct {
    FreeBlock *b;
    int n;
    int cap;
} FreeList;

#define PLAN_FAIL 0xFFFFFFFFu

static uint32_t round16(uint32_t v) { return (v + 15u) & ~15u; }

static int fl_reserve(FreeList *fl, int need) {
    if (need <= fl->cap) return 0;
    int cap = fl->cap ? fl->cap * 2 : 64;
    while (cap < need) cap *= 2;
    FreeBlock *nb = (FreeBlock *)realloc(fl->b, (size_t)cap * sizeof(FreeBlock));
    if (!nb) return -1;
    fl->b = nb;
    fl->cap = cap;
    return 0;
}

static uint32_t fl_alloc(FreeList *fl, uint32_t size) {
    if (size == 0) return 0;
    size = round16(size);
    int best = -1;
    for (int i = 0; i < fl->n; i++) {
        if (fl->b[i].size >= size && (best < 0 || fl->b[i].size < fl->b[best].size)) best = i;
    }
    if (best < 0) return PLAN_FAIL;
    uint32_t off = fl->b[best].offset;
    if (fl->b[best].size == size) {
        memmove(&fl->b[best], &fl->b[best + 1], (size_t)(fl->n - best - 1) * sizeof(FreeBlock));
        fl->n--;
    } else {
        fl->b[best].offset += size;
        fl->b[best].size -= size;
    }
    return off;
}

static int fl_release(FreeList *fl, uint32_t offset, uint32_t size) {
    if (size == 0) return 0;
    size = round16(size);
    if (fl_reserve(fl, fl->n + 1)) return -1;
    int pos = 0;
    while (pos < fl->n && fl->b[pos].offset < offset) pos++;
    memmove(&fl->b[pos + 1], &fl->b[pos], (size_t)(fl->n - pos) * sizeof(FreeBlock));
    fl->b[pos].offset = offset;
    fl->b[pos].size = size;
    fl->n++;
    /* merge with the successor */
    if (pos + 1 < fl->n && fl->b[pos].offset + fl->b[pos].size == fl->b[pos + 1].offset) {
        fl->b[pos].size += fl->b[pos + 1].size;
        memmove(&fl->b[pos + 1], &fl->b[pos + 2], (size_t)(fl->n - pos - 2) * sizeof(FreeBlock));
        fl->n--;
    }
    /* merge with the predecessor */
    if (pos > 0 && fl->b[pos - 1].offset + fl->b[pos - 1].size == fl->b[pos].offset) {
        fl->b[pos - 1].size += fl->b[pos].size;
        memmove(&fl->b[pos], &fl->b[pos + 1], (size_t)(fl->n - pos - 1) * sizeof(FreeBlock));
        fl->n--;
    }
    return 0;
}

static int place(FreeList *fl, SpinnTensor *t, uint32_t *peak) {
    t->offset = fl_alloc(fl, t->size);
    if (t->offset == PLAN_FAIL) return SPINN_MEM_ERR_NOMEM;
    uint32_t end = t->offset + round16(t->size);
    if (end > *peak) *peak = end;
    return 0;
}

int spinn_plan_memory(SpinnContext *ctx, uint32_t max_arena_bytes) {
    if (!ctx || !ctx->tensors || !ctx->nodes) return SPINN_MEM_ERR_NULL;
    FreeList fl = {0};
    uint8_t *remaining = (uint8_t *)malloc(ctx->num_tensors ? ctx->num_tensors : 1);
    uint8_t *is_output = (uint8_t *)calloc(ctx->num_tensors ? ctx->num_tensors : 1, 1);
    int rc = 0;
    uint32_t peak = 0;
    if (!remaining || !is_output || fl_reserve(&fl, 1)) {
        rc = SPINN_MEM_ERR_INTERNAL;
        goto done;
    }
    fl.b[0].offset = 0;
    fl.b[0].size = max_arena_bytes > 0 ? max_arena_bytes : 0xFFFFFFFFu;
    fl.n = 1;
    for (uint32_t i = 0; i < ctx->num_tensors; i++) remaining[i] = ctx->tensors[i].ref_count;
    for (int i = 0; i < ctx->header.num_outputs && i < 16; i++) {
        if (ctx->output_ids[i] < ctx->num_tensors) is_output[ctx->output_ids[i]] = 1;
    }

    for (int i = 0; i < ctx->header.num_inputs && i < 16; i++) {
        uint16_t id = ctx->input_ids[i];
        if (id >= ctx->num_tensors) continue;
        SpinnTensor *t = &ctx->tensors[id];
        if (t->is_weight || t->size == 0) continue;
        if ((rc = place(&fl, t, &peak)) != 0) goto done;
    }
    for (uint32_t n = 0; n < ctx->num_nodes; n++) {
        SpinnNode *node = &ctx->nodes[n];
        for (int j = 0; j < node->num_outputs; j++) {
            uint16_t id = node->output_ids[j];
            if (id >= ctx->num_tensors) continue;
            SpinnTensor *t = &ctx->tensors[id];
            if (t->is_weight || t->size == 0) continue;
            if ((rc = place(&fl, t, &peak)) != 0) goto done;
        }
        for (int j = 0; j < node->num_inputs; j++) {
            uint16_t id = node->input_ids[j];
            if (id >= ctx->num_tensors) continue;
            SpinnTensor *t = &ctx->tensors[id];
            if (t->is_weight || t->size == 0 || is_output[id]) continue;
            if (remaining[id] > 0 && --remaining[id] == 0) {
                if (fl_release(&fl, t->offset, t->size)) {
                    rc = SPINN_MEM_ERR_INTERNAL;
                    goto done;
                }
            }
        }
    }
    ctx->arena.peak_usage = peak;
    rc = peak > 0x7FFFFFFFu ? 0x7FFFFFFF : (int)peak;
done:
    free(fl.b);
    free(remaining);
    free(is_output);
    return rc;
}
