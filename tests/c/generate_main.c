/* generate_main.c -- a caller written against the reference's public API
 * (dnn_ctx_init, dnn_seed, decoder_lm_create, module_parameters,
 * decoder_lm_init_weights, decoder_lm_enable_rope, decoder_lm_generate), built
 * against include/dnn and linked with libdnn_amd.so.  It prints the weight
 * hashes and the generated ids as JSON so the tests can compare them with the
 * fixtures the reference itself wrote.
 *
 *   generate_main <V> <D> <L> <H> <F> <max_seq> <seed> <init> <prompt_seed> <P> <new> [temp] [use_cache]
 *   init: synthetic (N(0,0.02) on every non-gamma parameter) | gpt2 | create
 *   new = 0: no generation (no device use) -- prints the weights and the prompt
 */
#include "dnn/dnn.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static unsigned long long fnv(const void *p, size_t n) {
    const unsigned char *b = p;
    unsigned long long h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}

int main(int argc, char **argv) {
    if (argc < 12) { fprintf(stderr, "usage: see source\n"); return 2; }
    int V = atoi(argv[1]), D = atoi(argv[2]), L = atoi(argv[3]), H = atoi(argv[4]), F = atoi(argv[5]);
    int max_seq = atoi(argv[6]);
    unsigned long long seed = strtoull(argv[7], 0, 10);
    const char *init = argv[8];
    unsigned long long pseed = strtoull(argv[9], 0, 10);
    int P = atoi(argv[10]), NEW = atoi(argv[11]);
    float temp = argc > 12 ? (float)atof(argv[12]) : 0.0f;
    int use_cache = argc > 13 ? atoi(argv[13]) : 1;

    dnn_ctx ctx;
    size_t need = (size_t)(V * D + L * (4 * D * D + 3 * D * F + 8 * D + 2 * F) + 4 * V) * 4 + (size_t)max_seq * D * 4 + (64 << 20);
    if (dnn_ctx_init(&ctx, need, 16 << 20, 64 << 20)) return 1;
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx.params, V, D, L, H, D / H, F);
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    if (strcmp(init, "synthetic") == 0) {
        for (int i = 0; i < n; i++) {
            int gamma = ps[i] == lm->norm->weight;
            for (int l = 0; l < L; l++) gamma |= ps[i] == lm->blocks[l]->attn_norm->weight || ps[i] == lm->blocks[l]->ffn_norm->weight;
            if (gamma) continue;
            float *d = tensor_data_ptr(ps[i]);
            for (int j = 0; j < tensor_numel(ps[i]); j++) d[j] = dnn_rng_normal(dnn_get_rng()) * 0.02f;
        }
    } else if (strcmp(init, "gpt2") == 0) {
        decoder_lm_init_weights(lm);
    }
    decoder_lm_enable_rope(ctx.params, lm, max_seq, 10000.0f);

    dnn_rng r = dnn_rng_seed(pseed);
    tensor *prompt = tensor_zeros_data(ctx.data, 2, (int[]){1, P});
    for (int i = 0; i < P; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, V);
    int n_out = P;
    int *out = (int *)prompt->data;
    if (NEW > 0) out = decoder_lm_generate(ctx.scratch, ctx.data, lm, prompt, NEW, temp, use_cache, &n_out);

    printf("{\"params\": [");
    for (int i = 0; i < n; i++) printf("%s\"%016llx\"", i ? "," : "", fnv(tensor_data_ptr(ps[i]), sizeof(float) * (size_t)tensor_numel(ps[i])));
    printf("], \"tokens\": [");
    for (int i = 0; i < n_out; i++) printf("%s%d", i ? "," : "", out[i]);
    printf("]}\n");
    dnn_ctx_destroy(&ctx);
    return 0;
}
