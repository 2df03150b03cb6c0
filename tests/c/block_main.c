/* block_main.c -- a caller of the reference's layer-level API, written the way
 * the reference's own callers drive it (gpt.c:306-375, vlm.c:497-565):
 * kv_cache_create per layer, embedding_forward / decoder_lm_token_embeds,
 * transformer_block_forward_cached(_ex), rms_norm_forward,
 * decoder_lm_lm_head_forward, decoder_lm_argmax_token, tensor_cat,
 * decoder_lm_forward, kv_cache_get_K/V.  Built against include/dnn and linked
 * with libdnn_amd.so; every block / norm / head call runs on the device.
 *
 *   block_main c1  <outdir>   C1 (seed 1, N(0,0.02)): token-by-token run of the
 *                             16-id prompt + 240 new, the multi-token prefill
 *                             variant (+8 steps), decoder_lm_forward over 24 ids
 *   block_main vlm <outdir>   12 N(0,1) prefix rows ++ 4 text ids, one
 *                             PREFIX_LM pass, 6 decode steps
 *
 * Prints the ids as JSON; the logits go to <outdir>/<name>.f32. */
#include "dnn/dnn.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void save(const char *dir, const char *name, const float *p, size_t n) {
    char path[1024];
    snprintf(path, sizeof path, "%s/%s.f32", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, sizeof(float), n, f) != n) { perror(path); exit(1); }
    fclose(f);
}

/* A 4-D view (the kv_cache_get_K/V slices are strided) written out packed. */
static void save_view(const char *dir, const char *name, const tensor *t) {
    const int *n = t->shape;
    float *buf = malloc(sizeof(float) * (size_t)n[0] * n[1] * n[2] * n[3]), *o = buf;
    for (int a = 0; a < n[0]; a++)
        for (int b = 0; b < n[1]; b++)
            for (int c = 0; c < n[2]; c++)
                for (int d = 0; d < n[3]; d++)
                    *o++ = ((const float *)t->data)[t->offset + (size_t)a * t->strides[0] + (size_t)b * t->strides[1] +
                                                    (size_t)c * t->strides[2] + (size_t)d * t->strides[3]];
    save(dir, name, buf, (size_t)(o - buf));
    free(buf);
}

static void ints(const char *key, const int *v, int n, int last) {
    printf("\"%s\": [", key);
    for (int i = 0; i < n; i++) printf("%s%d", i ? "," : "", v[i]);
    printf("]%s", last ? "" : ", ");
}

static decoder_lm *synthetic(dnn_ctx *ctx, unsigned long long seed, int V, int D, int L, int H, int F, int max_seq) {
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx->params, V, D, L, H, D / H, F);
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    for (int i = 0; i < n; i++) {
        int gamma = ps[i] == lm->norm->weight;
        for (int l = 0; l < L; l++) gamma |= ps[i] == lm->blocks[l]->attn_norm->weight || ps[i] == lm->blocks[l]->ffn_norm->weight;
        if (gamma) continue;
        float *d = tensor_data_ptr(ps[i]);
        for (int j = 0; j < tensor_numel(ps[i]); j++) d[j] = dnn_rng_normal(dnn_get_rng()) * 0.02f;
    }
    decoder_lm_enable_rope(ctx->params, lm, max_seq, 10000.0f);
    return lm;
}

/* One decode step of id through every layer; logits row into lg. */
static int step(dnn_ctx *ctx, decoder_lm *lm, kv_cache **c, tensor *one, int id, float *lg) {
    ((int *)one->data)[0] = id;
    tensor *e = embedding_forward(ctx->scratch, NULL, lm->embed, one);
    tensor *h = tensor_reshape(ctx->scratch, e, 3, (int[]){1, 1, lm->d_model});
    for (int i = 0; i < lm->n_layers; i++) h = transformer_block_forward_cached(ctx->scratch, lm->blocks[i], h, c[i]);
    h = rms_norm_forward(ctx->scratch, lm->norm, h);
    tensor *l = decoder_lm_lm_head_forward(ctx->scratch, lm, h);
    memcpy(lg, tensor_data_ptr(l), sizeof(float) * lm->vocab_size);
    mem_pool_reset(ctx->scratch);
    return decoder_lm_argmax_token(lg, lm->vocab_size);
}

static int run_c1(dnn_ctx *ctx, const char *dir) {
    const int V = 128, D = 256, L = 4, H = 4, P = 16, NEW = 240;
    decoder_lm *lm = synthetic(ctx, 1, V, D, L, H, 683, 256);
    int prompt[16], out[256];
    dnn_rng r = dnn_rng_seed(101);
    for (int i = 0; i < P; i++) prompt[i] = dnn_rng_uniform_int(&r, V);
    dnn_grad_ctx g = dnn_no_grad_enter();
    printf("{");

    /* token by token: the prompt one id per call (logits only for the last), then greedy */
    {
        size_t mark = mem_pool_mark(ctx->data);
        kv_cache *c[4];
        for (int i = 0; i < L; i++) c[i] = kv_cache_create(ctx->data, 1, H, P + NEW, D / H);
        tensor *one = tensor_zeros_data(ctx->data, 1, (int[]){1});
        float *lg = malloc(sizeof(float) * (size_t)(NEW + 1) * V);
        memcpy(out, prompt, sizeof prompt);
        int cur = P, n = 0;
        for (int t = 0; cur < P + NEW; t++) {
            const int feed = t < P ? out[t] : out[cur - 1];
            const int id = step(ctx, lm, c, one, feed, lg + (size_t)n * V);
            if (t < P - 1) continue;
            n++;
            out[cur++] = id;
            if (id == TOKENIZER_EOS_ID) break;
        }
        save(dir, "c1_logits", lg, (size_t)n * V);
        ints("c1_tokens", out, cur, 0);
        /* the last layer's cache as kv_cache_get_K/V hand it to a host caller */
        tensor *K = kv_cache_get_K(ctx->scratch, c[L - 1]);
        tensor *Vt = kv_cache_get_V(ctx->scratch, c[L - 1]);
        printf("\"c1_cache_shape\": [%d,%d,%d,%d], ", K->shape[0], K->shape[1], K->shape[2], K->shape[3]);
        save_view(dir, "c1_K3", K);
        save_view(dir, "c1_V3", Vt);
        mem_pool_reset(ctx->scratch);
        free(lg);
        mem_pool_release(ctx->data, mark);
    }

    /* multi-token cached prefill of the prompt (N_new = P in one call per layer), then 8 steps */
    {
        size_t mark = mem_pool_mark(ctx->data);
        kv_cache *c[4];
        for (int i = 0; i < L; i++) c[i] = kv_cache_create(ctx->data, 1, H, 64, D / H);
        tensor *idp = tensor_zeros_data(ctx->data, 2, (int[]){1, P});
        memcpy(idp->data, prompt, sizeof prompt);
        tensor *h = decoder_lm_token_embeds(ctx->scratch, lm, idp);
        for (int i = 0; i < L; i++) h = transformer_block_forward_cached(ctx->scratch, lm->blocks[i], h, c[i]);
        h = rms_norm_forward(ctx->scratch, lm->norm, h);
        tensor *l = decoder_lm_lm_head_forward(ctx->scratch, lm, h);
        float pre[9 * 128];
        memcpy(pre, tensor_data_ptr(l) + (size_t)(P - 1) * V, sizeof(float) * V);
        int seq[9];
        seq[0] = decoder_lm_argmax_token(pre, V);
        mem_pool_reset(ctx->scratch);
        tensor *one = tensor_zeros_data(ctx->data, 1, (int[]){1});
        for (int s = 1; s < 9; s++) seq[s] = step(ctx, lm, c, one, seq[s - 1], pre + s * V);
        save(dir, "c1_prefill_logits", pre, 9 * 128);
        ints("c1_prefill_tokens", seq, 9, 0);
        mem_pool_release(ctx->data, mark);
    }

    /* decoder_lm_forward over the first 24 ids of the run */
    {
        tensor *ids = tensor_zeros_data(ctx->data, 2, (int[]){1, 24});
        memcpy(ids->data, out, sizeof(int) * 24);
        tensor *fl = decoder_lm_forward(ctx->scratch, lm, ids);
        save(dir, "c1_full24_logits", tensor_data_ptr(fl), 24 * 128);
        mem_pool_reset(ctx->scratch);
    }
    printf("\"done\": 1}\n");
    dnn_no_grad_exit(g);
    return 0;
}

static int run_vlm(dnn_ctx *ctx, const char *dir) {
    const int V = 96, D = 128, L = 2, H = 2, I = 12, T = 4, NS = 6;
    decoder_lm *lm = synthetic(ctx, 5, V, D, L, H, 256, 64);
    float *emb = malloc(sizeof(float) * I * D);
    dnn_rng r = dnn_rng_seed(505);
    for (int i = 0; i < I * D; i++) emb[i] = dnn_rng_normal(&r);
    int txt[4];
    for (int i = 0; i < T; i++) txt[i] = dnn_rng_uniform_int(&r, V);
    kv_cache *c[2];
    for (int i = 0; i < L; i++) c[i] = kv_cache_create(ctx->data, 1, H, I + T + NS, D / H);
    dnn_grad_ctx g = dnn_no_grad_enter();
    tensor *img = tensor_zeros(ctx->data, 3, (int[]){1, I, D}, 0);
    memcpy(tensor_data_ptr(img), emb, sizeof(float) * I * D);
    tensor *tid = tensor_zeros_data(ctx->data, 2, (int[]){1, T});
    memcpy(tid->data, txt, sizeof txt);
    tensor *te = decoder_lm_token_embeds(ctx->scratch, lm, tid);
    tensor *h = tensor_cat(ctx->scratch, img, te, 1);
    for (int i = 0; i < L; i++) h = transformer_block_forward_cached_ex(ctx->scratch, lm->blocks[i], h, c[i], ATTENTION_PREFIX_LM, I);
    h = rms_norm_forward(ctx->scratch, lm->norm, h);
    tensor *l = decoder_lm_lm_head_forward(ctx->scratch, lm, h);
    float *all = malloc(sizeof(float) * (I + T + NS) * V);
    memcpy(all, tensor_data_ptr(l), sizeof(float) * (I + T) * V);
    int seq[7];
    seq[0] = decoder_lm_argmax_token(all + (I + T - 1) * V, V);
    mem_pool_reset(ctx->scratch);
    tensor *one = tensor_zeros_data(ctx->data, 1, (int[]){1});
    for (int s = 1; s <= NS; s++) seq[s] = step(ctx, lm, c, one, seq[s - 1], all + (I + T + s - 1) * V);
    dnn_no_grad_exit(g);
    save(dir, "vlm_logits", all, (size_t)(I + T + NS) * V);
    printf("{");
    ints("vlm_tokens", seq, NS + 1, 1);
    printf("}\n");
    free(emb);
    free(all);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 3) { fprintf(stderr, "usage: block_main c1|vlm <outdir>\n"); return 2; }
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, 64 << 20, 64 << 20, 64 << 20)) return 1;
    int rc = strcmp(argv[1], "c1") == 0 ? run_c1(&ctx, argv[2]) : run_vlm(&ctx, argv[2]);
    dnn_ctx_destroy(&ctx);
    return rc;
}
