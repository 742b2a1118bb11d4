/*
 * main.c - `spinn_run model.ennf [runs] [--max-arena=SIZE] [--graph]` on the GPU.
 *
 * Same driver protocol as the reference CLI (SPINN/run_time/main.c:17-139):
 * load, plan (optionally capped), synthetic input x[i] = i/1000, 3 warm-up
 * runs when runs > 1, then best / average wall time of spinn_run (including
 * the host->device input copy, the device->host output copy and the final
 * stream synchronisation), the "SPINN Result:" line and the SPINN_DUMP
 * binary dump of every model output.
 */
#include "spinn_host.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1000.0 + ts.tv_nsec / 1e6;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        printf("Usage: %s <model.ennf> [num_runs] [--max-arena=SIZE] [--graph]\n", argv[0]);
        printf("  SIZE examples: 4M, 16M, 64M, 256M (0 = unlimited)\n");
        return 1;
    }
    int runs = 1, graph = 0;
    uint32_t max_arena = 0;
    for (int i = 2; i < argc; i++) {
        if (strncmp(argv[i], "--max-arena=", 12) == 0) {
            char *end = NULL;
            unsigned long v = strtoul(argv[i] + 12, &end, 10);
            if (end && (*end == 'K' || *end == 'k')) v *= 1024ul;
            else if (end && (*end == 'M' || *end == 'm')) v *= 1024ul * 1024ul;
            else if (end && (*end == 'G' || *end == 'g')) v *= 1024ul * 1024ul * 1024ul;
            max_arena = (uint32_t)v;
        } else if (strcmp(argv[i], "--graph") == 0) {
            graph = 1;
        } else {
            runs = atoi(argv[i]);
        }
    }
    if (runs < 1) runs = 1;
    const int warmup = runs > 1 ? 3 : 0;

    double t0 = now_ms();
    SpinnContext *ctx = spinn_load(argv[1]);
    if (!ctx) {
        fprintf(stderr, "Failed to load model\n");
        return 1;
    }
    double t_load = now_ms() - t0;
    t0 = now_ms();
    int rc = spinn_plan(ctx, max_arena);
    if (rc < 0) {
        if (rc == SPINN_MEM_ERR_NOMEM) fprintf(stderr, "Memory planning failed: Arena peak exceeds limit (%u bytes)\n", max_arena);
        else fprintf(stderr, "Failed to plan memory: %d\n", rc);
        spinn_free(ctx);
        return 1;
    }
    double t_plan = now_ms() - t0;
    if (graph) spinn_set_graph_mode(ctx, 1);

    SpinnTensor *tin = &ctx->tensors[ctx->input_ids[0]];
    SpinnTensor *tout = &ctx->tensors[ctx->output_ids[0]];
    float *in = (float *)malloc(tin->size ? tin->size : 4);
    float *out = (float *)malloc(tout->size ? tout->size : 4);
    if (!in || !out) return 1;
    for (uint32_t i = 0; i < tin->elem_count; i++) in[i] = (float)i / 1000.0f;
    if (runs > 1) {
        fprintf(stderr, "Load: %.1fms, Plan: %.1fms\n", t_load, t_plan);
        fprintf(stderr, "Warmup: %d, Runs: %d\n", warmup, runs);
    }
    for (int i = 0; i < warmup; i++) spinn_run(ctx, in, out);
    double best = 1e30, total = 0;
    for (int i = 0; i < runs; i++) {
        t0 = now_ms();
        rc = spinn_run(ctx, in, out);
        double dt = now_ms() - t0;
        if (rc < 0) {
            fprintf(stderr, "Inference failed: %d (%s) at node %d\n", rc, spinn_hip_error_string(rc),
                    ctx->last_error_node);
            break;
        }
        if (dt < best) best = dt;
        total += dt;
        if (runs > 1) fprintf(stderr, "  Run %d: %.3fms\n", i + 1, dt);
    }
    if (runs > 1) fprintf(stderr, "Best: %.3fms, Avg: %.3fms\n", best, total / runs);
    printf("SPINN Result: ");
    for (uint32_t i = 0; i < tout->elem_count; i++) printf("%.6f ", out[i]);
    printf("\n");
    const char *dump = getenv("SPINN_DUMP");
    if (dump && dump[0] != '0') {
        FILE *f = fopen(dump, "wb");
        if (f) {
            for (int oi = 0; oi < ctx->header.num_outputs && oi < 16; oi++) {
                SpinnTensor *to = &ctx->tensors[ctx->output_ids[oi]];
                if (!to->data || to->size == 0) continue;
                void *h = malloc(to->size);
                if (h && spinn_tensor_download(ctx, to->id, h, to->size) == 0) fwrite(h, 1, to->size, f);
                free(h);
            }
            fclose(f);
            fprintf(stderr, "Dumped %d outputs to %s\n", ctx->header.num_outputs, dump);
        }
    }
    free(in);
    free(out);
    spinn_profile_dump();
    spinn_free(ctx);
    return rc < 0 ? 1 : 0;
}
