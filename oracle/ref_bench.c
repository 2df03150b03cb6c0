/* ref_bench.c -- times the REAL reference's decode token loop (decoder_lm_generate
 * with use_cache=1, greedy) on the host CPU: bench.py's cpu_baseline leg.
 * Test infrastructure; built by oracle/Makefile against the reference's headers
 * into oracle/_ref/ref_bench (never shipped as product).
 *
 *   ref_bench V D L H F max_seq seed prompt_len new_tokens
 * Prints one JSON line: tokens, seconds for the generation loop, tok/s. */
#include "dnn.h"
#include "gpt.h"
#include <stdio.h>
#include <stdlib.h>
#include <time.h>

static double now(void) { struct timespec t; clock_gettime(CLOCK_MONOTONIC, &t); return t.tv_sec + 1e-9 * t.tv_nsec; }

int main(int argc, char **argv) {
    if (argc < 10) return 2;
    int V = atoi(argv[1]), D = atoi(argv[2]), L = atoi(argv[3]), H = atoi(argv[4]), F = atoi(argv[5]);
    int max_seq = atoi(argv[6]), P = atoi(argv[8]), NEW = atoi(argv[9]);
    unsigned long long seed = strtoull(argv[7], 0, 10);
    dnn_ctx ctx;
    size_t params = (size_t)(V * D + L * (4 * D * D + 3 * D * F + 8 * D + 2 * F) + 4 * V) * 4 + ((size_t)64 << 20);
    if (dnn_ctx_init(&ctx, params, (size_t)256 << 20, (size_t)512 << 20)) return 1;
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx.params, V, D, L, H, D / H, F);
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    for (int i = 0; i < n; i++) {
        if (ps[i] == lm->norm->weight) continue;
        int gamma = 0;
        for (int l = 0; l < L; l++) gamma |= ps[i] == lm->blocks[l]->attn_norm->weight || ps[i] == lm->blocks[l]->ffn_norm->weight;
        if (gamma) continue;
        float *d = tensor_data_ptr(ps[i]);
        for (int j = 0; j < tensor_numel(ps[i]); j++) d[j] = dnn_rng_normal(dnn_get_rng()) * 0.02f;
    }
    decoder_lm_enable_rope(ctx.params, lm, max_seq, 10000.0f);
    dnn_rng r = dnn_rng_seed(seed + 100);
    tensor *prompt = tensor_zeros_data(ctx.data, 2, (int[]){1, P});
    for (int i = 0; i < P; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, V);
    /* the timed call covers prompt + generation; report both the whole call and
     * the generation-only rate measured as (whole - prompt-only call) */
    int n_out;
    double t0 = now();
    decoder_lm_generate(ctx.scratch, ctx.data, lm, prompt, 1, 0.0f, 1, &n_out);
    double t_prompt = now() - t0;
    mem_pool_reset(ctx.scratch);
    t0 = now();
    decoder_lm_generate(ctx.scratch, ctx.data, lm, prompt, NEW, 0.0f, 1, &n_out);
    double t_all = now() - t0;
    int generated = n_out - P;
    double t_gen = t_all - t_prompt;
    printf("{\"tokens\": %d, \"seconds_total\": %.6f, \"seconds_prompt\": %.6f, \"tok_per_s\": %.6f}\n",
           generated, t_all, t_prompt, (generated - 1) / t_gen);
    return 0;
}
