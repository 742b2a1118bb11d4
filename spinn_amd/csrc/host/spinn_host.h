/*
 * spinn_host.h - internal declarations of the C host runtime.
 */
#ifndef SPINN_AMD_HOST_H
#define SPINN_AMD_HOST_H

#include "../../../include/spinn_runtime.h"
#include "../../../include/spinn_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Execution state the operator kernels launch with. The SpinnOpKernel
 * signature (SPINN/run_time/spinn_ops.h:31-33) carries no context, so the
 * runtime publishes the stream and the shared workspace here for the duration
 * of a run; outside spinn_run the operators use the null stream and a
 * library-owned workspace that grows on first need. */
typedef struct {
    void *stream;
    void *workspace;
    size_t workspace_bytes;
    int preparing; /* 1 while spinn_plan runs the prepare pass: pack weights, size workspace, launch nothing */
    size_t prepare_ws_need;
    int prepare_error;
    int conv_policy; /* SPINN_CONV_POLICY_* of the context being planned / run */
    int matmul_transposed; /* bit 0 / 1: the MatMul being dispatched gets operand A / B as its transpose */
    float matmul_alpha;    /* scale of the MatMul being dispatched (1 unless a Mul was folded into it) */
} SpinnExec;

extern SpinnExec g_spinn_exec;

/* Ensure the fallback workspace has `bytes`; returns it or NULL. */
void *spinn_exec_workspace(size_t bytes);
void spinn_exec_release_fallback(void);

/* Operator kernels (registered in ops.c). */
int op_conv2d(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out);
int op_gemm(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out);
int op_matmul(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out);
int op_maxpool(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out);
int op_global_avg_pool(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out,
                       int n_out);
int op_reduce_mean(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out);
int op_copy_alias(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out);
#define SPINN_DECLARE_OP(name) \
    int name(SpinnTensor **in, int n_in, void *params, uint16_t params_size, SpinnTensor **out, int n_out)
SPINN_DECLARE_OP(op_add);
SPINN_DECLARE_OP(op_sub);
SPINN_DECLARE_OP(op_mul);
SPINN_DECLARE_OP(op_div);
SPINN_DECLARE_OP(op_relu);
SPINN_DECLARE_OP(op_sigmoid);
SPINN_DECLARE_OP(op_batch_norm);
SPINN_DECLARE_OP(op_softmax);
SPINN_DECLARE_OP(op_concat);
SPINN_DECLARE_OP(op_split);
SPINN_DECLARE_OP(op_transpose);
SPINN_DECLARE_OP(op_resize);
SPINN_DECLARE_OP(op_mod);
SPINN_DECLARE_OP(op_reduce_max);
SPINN_DECLARE_OP(op_topk);
SPINN_DECLARE_OP(op_gather_elements);
SPINN_DECLARE_OP(op_tile);
SPINN_DECLARE_OP(op_cast);

/* Build the conv descriptor exactly as op_conv2d reads its operands. */
int spinn_conv_desc_from_tensors(SpinnTensor **in, int n_in, const void *params, uint16_t params_size,
                                 SpinnTensor **out, SpinnHipConvDesc *d, const float **bias, const float **res);
int spinn_op_registered(uint16_t op_type);

/* Packed (re-laid-out) weight buffers and the layout each holds. */
int spinn_packed_alloc(void **dev, size_t bytes, int algo);
int spinn_packed_matches(const void *dev, size_t bytes, int algo);
void spinn_packed_release(void *dev);

/* Owner of packed weight buffers created by the operators (freed by spinn_free). */
void spinn_free_packed(SpinnContext *ctx);

#ifdef __cplusplus
}
#endif
#endif
