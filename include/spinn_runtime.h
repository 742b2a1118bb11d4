/*
 * spinn_runtime.h - host runtime API (load -> plan -> run) over an HBM arena.
 *
 * Same three-phase API, structs and return conventions as the reference runtime
 * (SPINN/run_time/spinn_runtime.h:25-144, spinn_ops.h:25-33,
 * spinn_memory_planner.h:17-33), so callers written against it (the CLI driver,
 * generated model code) compile unchanged. What differs is where memory lives:
 *
 *   - spinn_plan() places every activation at the planner's offset inside ONE
 *     device allocation (hipMalloc'd arena), instead of a calloc'd host arena
 *     (reference: SPINN/run_time/spinn_runtime.c:143-152);
 *   - weights are read once at plan time and uploaded into one device weight
 *     pool; SpinnTensor.data of a weight is its device address;
 *   - SpinnTensor.data is therefore always a DEVICE pointer, and the operator
 *     kernels registered behind spinn_dispatch_op() are HIP launches;
 *   - spinn_run() copies input 0 host->device, launches every node on the
 *     runtime's stream, copies output 0 device->host and synchronises. Passing
 *     NULL for input/output skips the copy, as in the reference, which lets a
 *     caller keep inputs resident in HBM.
 */
#ifndef SPINN_AMD_RUNTIME_H
#define SPINN_AMD_RUNTIME_H

#include <stdint.h>
#include <stddef.h>
#include <stdio.h>
#include "ennf_format.h"

#ifdef __cplusplus
extern "C" {
#endif

/* SPINN/run_time/spinn_runtime.h:25-40 */
typedef struct {
    uint16_t id;
    uint8_t dtype;
    uint8_t ndim;
    uint32_t dims[ENNF_MAX_DIMS];
    uint32_t elem_count;
    uint8_t is_weight;
    uint8_t ref_count;
    uint32_t size;      /* bytes = elem_count * dtype size */
    uint32_t offset;    /* arena offset from the planner */
    void *data;         /* device address: arena base + offset, or device weight copy */
    void *packed_data;  /* device address of an operator's re-laid-out weights (owned by the tensor) */
} SpinnTensor;

#define SPINN_MAX_IO 8

/* SPINN/run_time/spinn_runtime.h:47-57 */
typedef struct {
    uint16_t op_type;
    uint8_t num_inputs;
    uint8_t num_outputs;
    uint16_t input_ids[SPINN_MAX_IO];
    uint16_t output_ids[SPINN_MAX_IO];
    uint16_t params_size;
    void *params;
} SpinnNode;

/* SPINN/run_time/spinn_runtime.h:62-66; base is a device address here. */
typedef struct {
    uint8_t *base;
    size_t capacity;
    size_t peak_usage;
} SpinnArena;

/* SPINN/run_time/spinn_runtime.h:71-96, plus device-side fields at the end. */
typedef struct {
    ENNF_Header header;
    uint16_t input_ids[16];
    uint16_t output_ids[16];
    SpinnTensor *tensors;
    uint32_t num_tensors;
    SpinnNode *nodes;
    uint32_t num_nodes;
    SpinnArena arena;
    FILE *ennf_fp;
    uint32_t weight_base_offset;
    void **weight_cache;     /* host copies, filled lazily by spinn_get_weight() */
    uint32_t num_weights;
    uint16_t flags;
    /* device-side state */
    void *stream;            /* hipStream_t all nodes are launched on */
    uint8_t *weight_pool;    /* one device allocation holding every weight */
    size_t weight_pool_bytes;
    void *workspace;         /* device scratch shared by the operators (split-K partials) */
    size_t workspace_bytes;
    int last_error;          /* first non-zero operator return code of the last run */
    int last_error_node;     /* node index that returned it, or -1 */
    void *graph_exec;        /* hipGraphExec_t of the node loop when graph replay is on */
    int use_graph;
    void *prof_state;        /* per-node HIP events and times when SPINN_PROFILE=1 */
    int conv_policy;         /* SPINN_CONV_POLICY_* fixed at plan time */
    void *input_stage;       /* device copy of input 0 that spinn_run_resident restores from */
    int input_staged;        /* 1 once spinn_stage_input has filled input_stage */
    uint8_t *node_folded;    /* per node, set by spinn_plan: 1 when a consumer reads the node's input in its
                                place (a Transpose read transposed by its MatMul), so the node launches nothing */
    int32_t *node_tsrc;      /* per node, two entries set by spinn_plan: the tensor a MatMul reads transposed
                                as its operand A / B instead of that operand, or -1 */
    int32_t *node_tdst;      /* per node, set by spinn_plan: the tensor a MatMul writes instead of its output
                                (the output of a folded Mul by a constant scalar), or -1 */
    float *node_alpha;       /* per node: the scale a MatMul applies to its product (that scalar), else 1 */
} SpinnContext;

/* Which algorithm eligible 3x3 stride-1 convolutions use (spinn_set_conv_policy). */
#define SPINN_CONV_POLICY_AUTO 0     /* per-shape choice of the compute layer */
#define SPINN_CONV_POLICY_IGEMM 1    /* always the implicit GEMM */
#define SPINN_CONV_POLICY_WINOGRAD 2 /* Winograd wherever eligible (F(4x4,3x3) unless AUTO picked F(2x2,3x3)) */

/* Planner error codes (SPINN/run_time/spinn_memory_planner.h:17-20). */
#define SPINN_MEM_OK 0
#define SPINN_MEM_ERR_NULL -1
#define SPINN_MEM_ERR_NOMEM -2
#define SPINN_MEM_ERR_INTERNAL -3

/* Operator kernel signature and dispatcher (SPINN/run_time/spinn_ops.h:25-33). */
typedef int (*SpinnOpKernel)(SpinnTensor **in, int n_in, void *params, uint16_t params_size,
                             SpinnTensor **out, int n_out);
int spinn_dispatch_op(uint16_t op_type, SpinnTensor **inputs, int n_in, void *params,
                      uint16_t params_size, SpinnTensor **outputs, int n_out);

/* Public API (SPINN/run_time/spinn_runtime.h:107-144). */
SpinnContext *spinn_load(const char *path);
int spinn_plan(SpinnContext *ctx, uint32_t max_arena_bytes);
int spinn_run(SpinnContext *ctx, void *input_data, void *output_data);
void spinn_free(SpinnContext *ctx);
void spinn_profile_dump(void);
void *spinn_get_weight(SpinnContext *ctx, uint16_t tensor_id);

/* Static memory planner (SPINN/run_time/spinn_memory_planner.h:33). */
int spinn_plan_memory(SpinnContext *ctx, uint32_t max_arena_bytes);

/* ---- Extensions (no counterpart in the reference) ---- */

/* Copy host bytes into / out of a planned tensor (device memory); synchronous. */
int spinn_tensor_upload(SpinnContext *ctx, uint16_t tensor_id, const void *host, size_t bytes);
int spinn_tensor_download(SpinnContext *ctx, uint16_t tensor_id, void *host, size_t bytes);

/* Copy input 0 from the host into the context's device staging buffer (a
 * separate allocation made by spinn_plan, outside the arena); synchronous.
 * The staged copy stays untouched by the node loop. */
int spinn_stage_input(SpinnContext *ctx, const void *host, size_t bytes);

/* Device address of the staging buffer (NULL before spinn_plan), for callers
 * that produce input 0 on the device themselves; after writing it they call
 * spinn_stage_input(ctx, NULL, 0) to mark it filled. */
void *spinn_input_stage_ptr(SpinnContext *ctx);

/* One step with the input resident in HBM: copy the staged input 0 into its
 * arena region (device to device, on the runtime's stream), run the node loop
 * and leave the outputs in the arena; returns after the stream is idle.
 * The copy is what the reference's spinn_run does with its host input on
 * every call (SPINN/run_time/spinn_runtime.c:302-306): the planner hands the
 * input's arena region to later activations once its last consumer has run,
 * so a run that skips it computes on the previous run's activations.
 * Returns -1 when nothing has been staged. spinn_run(ctx, NULL, NULL) keeps
 * the reference's meaning (no copy at all). */
int spinn_run_resident(SpinnContext *ctx);

/* Capture the node loop into a HIP graph and replay it on later runs (1) or
 * launch every node individually (0, the default). */
int spinn_set_graph_mode(SpinnContext *ctx, int enable);

/* Set the conv algorithm policy; only before spinn_plan (weights are re-laid
 * out for the chosen algorithm at plan time). Returns -1 after plan. */
int spinn_set_conv_policy(SpinnContext *ctx, int policy);

/* Turn per-node HIP-event timing on or off (overrides SPINN_PROFILE). */
void spinn_set_profiling(int on);

/* Per-node device time of the last run when SPINN_PROFILE=1 (milliseconds,
 * from HIP events around each node). Returns the number of nodes written. */
int spinn_node_times(SpinnContext *ctx, float *ms_out, int max_nodes);

#ifdef __cplusplus
}
#endif
#endif /* SPINN_AMD_RUNTIME_H */
