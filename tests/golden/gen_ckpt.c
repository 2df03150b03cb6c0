/*
 * gen_ckpt.c -- writes a DNNM checkpoint with the REAL reference's module_save
 * (module.c:208-230; compiled from /root/reference/src into
 * oracle/_ref/libdnnref.so) and the greedy ids the reference generates from
 * it, into tests/golden/data/ckpt_small.dnnm and ckpt.json.  Dev container
 * only; the files are committed data.  Build + run: tests/golden/make_golden.sh
 *
 * Model: vocab 64, d_model 64, 2 layers, 1 head, d_ffn 96, seed 9,
 * decoder_lm_init_weights (GPT-2 style), RoPE for 64 positions.
 */
#include "dnn.h"
#include "gpt.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t fnv(const void *p, size_t n) {
    const unsigned char *b = p;
    uint64_t h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}

int main(void) {
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, (size_t)16 << 20, (size_t)16 << 20, (size_t)16 << 20)) return 1;
    dnn_seed(9);
    decoder_lm *lm = decoder_lm_create(ctx.params, 64, 64, 2, 1, 64, 96);
    decoder_lm_init_weights(lm);
    decoder_lm_enable_rope(ctx.params, lm, 64, 10000.0f);
    module_save(&lm->base, "tests/golden/data/ckpt_small.dnnm");
    FILE *J = fopen("tests/golden/data/ckpt.json", "w");
    if (!J) return 1;
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    fprintf(J, "{\"ckpt_params\": [");
    for (int i = 0; i < n; i++)
        fprintf(J, "%s\"%016llx\"", i ? "," : "",
                (unsigned long long)fnv(tensor_data_ptr(ps[i]), (size_t)tensor_numel(ps[i]) * 4));
    tensor *prompt = tensor_zeros_data(ctx.data, 2, (int[]){1, 5});
    dnn_rng r = dnn_rng_seed(909);
    for (int i = 0; i < 5; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, 64);
    int no;
    int *o = decoder_lm_generate(ctx.scratch, ctx.data, lm, prompt, 20, 0.0f, 1, &no);
    fprintf(J, "], \"ckpt_tokens\": [");
    for (int i = 0; i < no; i++) fprintf(J, "%s%d", i ? "," : "", o[i]);
    fprintf(J, "]}\n");
    fclose(J);
    dnn_ctx_destroy(&ctx);
    return 0;
}
