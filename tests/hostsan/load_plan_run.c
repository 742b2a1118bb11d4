/* load_plan_run.c - drive the C runtime's host code over .ennf files under
 * AddressSanitizer / UBSan (built with hip_stub.c by tests/test_host_sanitizers.py).
 *
 * For each file: spinn_load; if it loads, spinn_plan, then spinn_run eagerly
 * and in graph mode (the stub's graph capture fails, exercising that error
 * path), then spinn_free. Prints one line per file: the load / plan / run
 * return codes and what the plan folded (view outputs sharing their input's
 * bytes, Transposes read by their MatMul, scalar Muls taken as MatMul alpha).
 * Any sanitizer report aborts the process with a non-zero exit.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "spinn_runtime.h"

int main(int argc, char **argv) {
    for (int i = 1; i < argc; i++) {
        SpinnContext *ctx = spinn_load(argv[i]);
        if (!ctx) {
            printf("%s load=fail\n", argv[i]);
            continue;
        }
        int plan = spinn_plan(ctx, 0);
        int run = 99, run_graph = 99;
        int views = 0, transposes = 0, scales = 0;
        if (plan == 0) {
            for (uint32_t k = 0; k < ctx->num_nodes; k++) {
                const SpinnNode *nd = &ctx->nodes[k];
                const uint16_t op = nd->op_type;
                if ((op == ENNF_OP_Reshape || op == ENNF_OP_Flatten || op == ENNF_OP_Identity ||
                     op == ENNF_OP_Unsqueeze) &&
                    nd->num_inputs >= 1 && nd->num_outputs >= 1 &&
                    ctx->tensors[nd->input_ids[0]].data == ctx->tensors[nd->output_ids[0]].data)
                    views++;
                if (ctx->node_folded && ctx->node_folded[k] && op == ENNF_OP_Transpose) transposes++;
                if (ctx->node_tdst && ctx->node_tdst[k] >= 0) scales++;
            }
        }
        if (plan == 0) {
            /* spinn_run copies tensor input_ids[0] in and output_ids[0] out
             * (both validated ids, 0 when the file lists none) */
            size_t in_bytes = ctx->tensors[ctx->input_ids[0]].size;
            size_t out_bytes = ctx->tensors[ctx->output_ids[0]].size;
            void *in = calloc(1, in_bytes + 16), *out = calloc(1, out_bytes + 16);
            run = spinn_run(ctx, in, out);
            spinn_set_graph_mode(ctx, 1);
            run_graph = spinn_run(ctx, in, out);
            free(in);
            free(out);
        }
        printf("%s load=ok plan=%d run=%d run_graph=%d views=%d transposes=%d scales=%d\n", argv[i], plan, run,
               run_graph, views, transposes, scales);
        spinn_free(ctx);
    }
    return 0;
}
