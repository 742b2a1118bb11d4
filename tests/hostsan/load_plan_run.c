/* load_plan_run.c - drive the C runtime's host code over .ennf files under
 * AddressSanitizer / UBSan (built with hip_stub.c by tests/test_host_sanitizers.py).
 *
 * For each file: spinn_load; if it loads, spinn_plan, then spinn_run eagerly
 * and in graph mode (the stub's graph capture fails, exercising that error
 * path), then spinn_free. Prints one line per file: the load / plan / run
 * return codes. Any sanitizer report aborts the process with a non-zero exit.
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
        printf("%s load=ok plan=%d run=%d run_graph=%d\n", argv[i], plan, run, run_graph);
        spinn_free(ctx);
    }
    return 0;
}
