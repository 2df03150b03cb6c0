/* ckpt_main.c -- module_save / module_load (module.c:174-339) from a caller of
 * the reference's API, against a DNNM file the reference itself wrote
 * (tests/golden/gen_ckpt.c).
 *
 *   ckpt_main load <ckpt> <tmpfile>   a model of other weights loads the file
 *                                     (strict); its parameters' hashes; then
 *                                     save + load into a third model
 *   ckpt_main gen <ckpt>              greedy generate on the model's own weights,
 *                                     module_load, generate again (the device
 *                                     mirror must follow the new weights)
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

static decoder_lm *model(dnn_ctx *ctx, unsigned long long seed) {
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx->params, 64, 64, 2, 1, 64, 96);
    decoder_lm_init_weights(lm);
    decoder_lm_enable_rope(ctx->params, lm, 64, 10000.0f);
    return lm;
}

static void hashes(const char *key, decoder_lm *lm) {
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    printf("\"%s\": [", key);
    for (int i = 0; i < n; i++)
        printf("%s\"%016llx\"", i ? "," : "", fnv(tensor_data_ptr(ps[i]), sizeof(float) * (size_t)tensor_numel(ps[i])));
    printf("]");
}

static void gen(dnn_ctx *ctx, decoder_lm *lm, const char *key) {
    tensor *prompt = tensor_zeros_data(ctx->data, 2, (int[]){1, 5});
    dnn_rng r = dnn_rng_seed(909);
    for (int i = 0; i < 5; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, 64);
    int no;
    int *o = decoder_lm_generate(ctx->scratch, ctx->data, lm, prompt, 20, 0.0f, 1, &no);
    printf("\"%s\": [", key);
    for (int i = 0; i < no; i++) printf("%s%d", i ? "," : "", o[i]);
    printf("]");
}

int main(int argc, char **argv) {
    if (argc < 3) { fprintf(stderr, "usage: see source\n"); return 2; }
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, 16 << 20, 16 << 20, 16 << 20)) return 1;
    printf("{");
    if (strcmp(argv[1], "load") == 0 && argc > 3) {
        decoder_lm *a = model(&ctx, 1);
        hashes("before", a);
        module_load(&a->base, argv[2], 1);
        printf(", ");
        hashes("loaded", a);
        module_save(&a->base, argv[3]);
        decoder_lm *b = model(&ctx, 2);
        module_load(&b->base, argv[3], 1);
        printf(", ");
        hashes("reloaded", b);
    } else {
        decoder_lm *a = model(&ctx, 1);
        gen(&ctx, a, "own");
        module_load(&a->base, argv[2], 1);
        printf(", ");
        gen(&ctx, a, "loaded");
    }
    printf("}\n");
    dnn_ctx_destroy(&ctx);
    return 0;
}
