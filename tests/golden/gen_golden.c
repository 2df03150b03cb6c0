/*
 * gen_golden.c -- writes the golden fixtures in tests/golden/data/ by running the
 * REAL reference (masc-it/dnn.c compiled from /root/reference/src into
 * oracle/_ref/libdnnref.so by oracle/Makefile).  Runs only where /root/reference
 * exists (the dev container); the fixtures it writes are committed data.
 *
 * Build + run: tests/golden/make_golden.sh
 *
 * Everything goes through the reference's public C API (include/*.h there):
 * dnn_seed, decoder_lm_create, module_parameters, decoder_lm_enable_rope,
 * decoder_lm_generate, transformer_block_forward_cached(_ex), rms_norm_forward,
 * decoder_lm_lm_head_forward, decoder_lm_forward, tensor_* ops.
 */
#include "dnn.h"
#include "gpt.h"
#include "rope.h"
#include "norm.h"
#include "ops.h"
#include "multihead.h"
#include "autograd.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <time.h>

static const char *OUT = "tests/golden/data";
static FILE *J;            /* index.json */
static int first_key = 1;

static uint64_t fnv(const void *p, size_t n) {
    const unsigned char *b = p;
    uint64_t h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}

static void key(const char *k) { fprintf(J, "%s\n\"%s\": ", first_key ? "" : ",", k); first_key = 0; }
static void j_ints(const char *k, const int *v, int n) {
    key(k); fputc('[', J);
    for (int i = 0; i < n; i++) fprintf(J, "%s%d", i ? "," : "", v[i]);
    fputc(']', J);
}
static void j_floats(const char *k, const float *v, int n) {   /* exact: hex bit patterns */
    key(k); fputc('[', J);
    for (int i = 0; i < n; i++) { uint32_t u; memcpy(&u, &v[i], 4); fprintf(J, "%s%u", i ? "," : "", u); }
    fputc(']', J);
}
static void j_hash(const char *k, const void *p, size_t n) { key(k); fprintf(J, "\"%016llx\"", (unsigned long long)fnv(p, n)); }
static void j_num(const char *k, double v) { key(k); fprintf(J, "%.17g", v); }
static void bin(const char *name, const void *p, size_t n) {
    char path[512]; snprintf(path, sizeof path, "%s/%s", OUT, name);
    FILE *f = fopen(path, "wb"); fwrite(p, 1, n, f); fclose(f);
}

static double now(void) { struct timespec t; clock_gettime(CLOCK_MONOTONIC, &t); return t.tv_sec + 1e-9 * t.tv_nsec; }

/* Synthetic init used by every parity config: the reference's own create-time
 * draws, then every parameter except RMSNorm gammas <- N(0,1)*std in
 * module_parameters() order, from the same default stream. */
static decoder_lm *make_model(dnn_ctx *ctx, uint64_t seed, int V, int D, int L, int H, int F,
                              int max_seq, float std) {
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx->params, V, D, L, H, D / H, F);
    int n; tensor **ps = module_parameters(&lm->base, &n);
    for (int i = 0; i < n; i++) {
        int is_gamma = 0;
        if (lm->norm->weight == ps[i]) is_gamma = 1;
        for (int l = 0; l < L; l++)
            if (lm->blocks[l]->attn_norm->weight == ps[i] || lm->blocks[l]->ffn_norm->weight == ps[i]) is_gamma = 1;
        if (is_gamma) continue;
        float *d = tensor_data_ptr(ps[i]);
        int ne = tensor_numel(ps[i]);
        for (int j = 0; j < ne; j++) d[j] = dnn_rng_normal(dnn_get_rng()) * std;
    }
    decoder_lm_enable_rope(ctx->params, lm, max_seq, 10000.0f);
    return lm;
}

/* The reference's own GPT-2-style init (gpt.c:431-477): std 1/sqrt(D) gives
 * unit-scale logits and far more varied greedy runs than std 0.02. */
static decoder_lm *make_model_gpt2(dnn_ctx *ctx, uint64_t seed, int V, int D, int L, int H, int F,
                                   int max_seq) {
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx->params, V, D, L, H, D / H, F);
    decoder_lm_init_weights(lm);
    decoder_lm_enable_rope(ctx->params, lm, max_seq, 10000.0f);
    return lm;
}

static void params_hash(const char *prefix, decoder_lm *lm) {
    int n; tensor **ps = module_parameters(&lm->base, &n);
    uint64_t *h = malloc(sizeof(uint64_t) * n);
    char k[128];
    key(prefix); fputc('[', J);
    for (int i = 0; i < n; i++) {
        h[i] = fnv(tensor_data_ptr(ps[i]), (size_t)tensor_numel(ps[i]) * 4);
        fprintf(J, "%s\"%016llx\"", i ? "," : "", (unsigned long long)h[i]);
    }
    fputc(']', J);
    snprintf(k, sizeof k, "%s_first4", prefix);
    key(k); fputc('[', J);
    for (int i = 0; i < n; i++) {
        float *d = tensor_data_ptr(ps[i]);
        for (int j = 0; j < 4 && j < tensor_numel(ps[i]); j++) { uint32_t u; memcpy(&u, &d[j], 4); fprintf(J, "%s%u", (i || j) ? "," : "", u); }
    }
    fputc(']', J);
    free(h);
}

static void prompt_ids(uint64_t seed, int V, int P, int *out) {
    dnn_rng r = dnn_rng_seed(seed);
    for (int i = 0; i < P; i++) out[i] = dnn_rng_uniform_int(&r, V);
}

/* The reference generate loop written out with its public per-layer API, so
 * the per-step logits can be recorded (same calls as gpt.c:306-375). */
static int manual_generate(dnn_ctx *ctx, decoder_lm *lm, const int *prompt, int P, int max_new,
                           int *out, float *logits_all, float *margins, uint64_t *hashes,
                           float *first8) {
    int V = lm->vocab_size, D = lm->d_model, max_len = P + max_new;
    size_t mark = mem_pool_mark(ctx->data);
    kv_cache **c = _mem_pool_alloc(ctx->data, sizeof(kv_cache*) * lm->n_layers, NULL);
    for (int i = 0; i < lm->n_layers; i++) c[i] = kv_cache_create(ctx->data, 1, lm->blocks[0]->n_heads, max_len, lm->blocks[0]->d_k);
    tensor *one = tensor_zeros_data(ctx->data, 1, (int[]){1});
    float *lg = malloc(sizeof(float) * V);
    memcpy(out, prompt, sizeof(int) * P);
    int cur = P, step = 0;
    dnn_grad_ctx g = dnn_no_grad_enter();
    for (int t = 0; cur < max_len; t++) {
        int feed = (t < P) ? out[t] : out[cur - 1];
        ((int*)one->data)[0] = feed;
        tensor *e = embedding_forward(ctx->scratch, NULL, lm->embed, one);
        tensor *h = tensor_reshape(ctx->scratch, e, 3, (int[]){1, 1, D});
        for (int i = 0; i < lm->n_layers; i++) h = transformer_block_forward_cached(ctx->scratch, lm->blocks[i], h, c[i]);
        if (t < P - 1) { mem_pool_reset(ctx->scratch); continue; }
        h = rms_norm_forward(ctx->scratch, lm->norm, h);
        tensor *l = decoder_lm_lm_head_forward(ctx->scratch, lm, h);
        memcpy(lg, tensor_data_ptr(l), sizeof(float) * V);
        mem_pool_reset(ctx->scratch);
        int id = decoder_lm_argmax_token(lg, V);
        if (logits_all) memcpy(logits_all + (size_t)step * V, lg, sizeof(float) * V);
        if (margins) {
            float second = -INFINITY;
            for (int i = 0; i < V; i++) if (i != id && lg[i] > second) second = lg[i];
            margins[step] = lg[id] - second;
        }
        if (hashes) hashes[step] = fnv(lg, sizeof(float) * V);
        if (first8) memcpy(first8 + (size_t)step * 8, lg, sizeof(float) * 8);
        step++;
        out[cur++] = id;
        if (id == TOKENIZER_EOS_ID) break;
    }
    dnn_no_grad_exit(g);
    mem_pool_release(ctx->data, mark);
    free(lg);
    return cur;
}

static void gen_rng(void) {
    uint64_t seeds[4] = {0, 1, 42, 12345};
    char k[64];
    for (int s = 0; s < 4; s++) {
        dnn_rng r = dnn_rng_seed(seeds[s]);
        float u[8], nrm[8]; int ii[8], jj[8];
        for (int i = 0; i < 8; i++) u[i] = dnn_rng_uniform(&r);
        for (int i = 0; i < 8; i++) nrm[i] = dnn_rng_normal(&r);
        for (int i = 0; i < 8; i++) ii[i] = dnn_rng_uniform_int(&r, 8192);
        for (int i = 0; i < 8; i++) jj[i] = dnn_rng_uniform_int(&r, 49);
        snprintf(k, sizeof k, "rng_%llu_uniform", (unsigned long long)seeds[s]); j_floats(k, u, 8);
        snprintf(k, sizeof k, "rng_%llu_normal", (unsigned long long)seeds[s]); j_floats(k, nrm, 8);
        snprintf(k, sizeof k, "rng_%llu_int8192", (unsigned long long)seeds[s]); j_ints(k, ii, 8);
        snprintf(k, sizeof k, "rng_%llu_int49", (unsigned long long)seeds[s]); j_ints(k, jj, 8);
        /* raw state after seeding */
        dnn_rng r0 = dnn_rng_seed(seeds[s]);
        snprintf(k, sizeof k, "rng_%llu_state", (unsigned long long)seeds[s]);
        key(k); fprintf(J, "[\"%016llx\",\"%016llx\"]", (unsigned long long)r0.s[0], (unsigned long long)r0.s[1]);
    }
    /* default thread-local stream before any dnn_seed: {1,2} */
}

/* Op-level fixtures on inputs drawn from a private stream (seed 777). */
static void gen_ops(dnn_ctx *ctx) {
    dnn_rng r = dnn_rng_seed(777);
    /* matmul_add, both layouts: a [2,3,37], w [37,53] / [53,37], b [53] */
    int M = 3, K = 37, N = 53;
    tensor *a = tensor_zeros(ctx->data, 3, (int[]){2, M, K}, 0);
    tensor *w = tensor_zeros(ctx->data, 2, (int[]){K, N}, 0);
    tensor *wt = tensor_zeros(ctx->data, 2, (int[]){N, K}, 0);
    tensor *b = tensor_zeros(ctx->data, 1, (int[]){N}, 0);
    float *ad = tensor_data_ptr(a), *wd = tensor_data_ptr(w), *wtd = tensor_data_ptr(wt), *bd = tensor_data_ptr(b);
    for (int i = 0; i < 2 * M * K; i++) ad[i] = dnn_rng_normal(&r);
    for (int i = 0; i < K * N; i++) wd[i] = dnn_rng_normal(&r);
    for (int i = 0; i < K * N; i++) wtd[i] = dnn_rng_normal(&r);
    for (int i = 0; i < N; i++) bd[i] = dnn_rng_normal(&r);
    dnn_grad_ctx g = dnn_no_grad_enter();
    tensor *y = tensor_matmul_add(ctx->scratch, a, w, 0, b);
    tensor *yt = tensor_matmul_add(ctx->scratch, a, wt, 1, b);
    j_floats("op_mm_a", ad, 2 * M * K); j_floats("op_mm_w", wd, K * N); j_floats("op_mm_wt", wtd, K * N);
    j_floats("op_mm_b", bd, N);
    j_floats("op_mm_y", tensor_data_ptr(y), 2 * M * N); j_floats("op_mm_yt", tensor_data_ptr(yt), 2 * M * N);

    /* rms_norm over d=768 and d=683 (odd: exercises the vector remainder) */
    int ds[2] = {768, 683};
    for (int t = 0; t < 2; t++) {
        int d = ds[t];
        tensor *x = tensor_zeros(ctx->data, 2, (int[]){3, d}, 0);
        tensor *gm = tensor_zeros(ctx->data, 1, (int[]){d}, 0);
        float *xd = tensor_data_ptr(x), *gd = tensor_data_ptr(gm);
        for (int i = 0; i < 3 * d; i++) xd[i] = dnn_rng_normal(&r) * 3.0f;
        for (int i = 0; i < d; i++) gd[i] = 1.0f + 0.1f * dnn_rng_normal(&r);
        tensor *yy = tensor_rms_norm(ctx->scratch, x, gm, 1e-5f);
        char k[64];
        snprintf(k, sizeof k, "op_rms%d_x", d); j_floats(k, xd, 3 * d);
        snprintf(k, sizeof k, "op_rms%d_g", d); j_floats(k, gd, d);
        snprintf(k, sizeof k, "op_rms%d_y", d); j_floats(k, tensor_data_ptr(yy), 3 * d);
    }

    /* rope on [1,2,5,64] at positions 7..11 of a 1088-row table */
    tensor *fc, *fs;
    tensor_rope_freqs_init(ctx->data, &fc, &fs, 64, 1088, 10000.0f);
    j_hash("rope_cos_hash", tensor_data_ptr(fc), 1088 * 32 * 4);
    j_hash("rope_sin_hash", tensor_data_ptr(fs), 1088 * 32 * 4);
    j_floats("rope_cos_row1000", tensor_data_ptr(fc) + 1000 * 32, 32);
    j_floats("rope_sin_row1000", tensor_data_ptr(fs) + 1000 * 32, 32);
    tensor *xr = tensor_zeros(ctx->data, 4, (int[]){1, 2, 5, 64}, 0);
    float *xrd = tensor_data_ptr(xr);
    for (int i = 0; i < 640; i++) xrd[i] = dnn_rng_normal(&r);
    j_floats("op_rope_x", xrd, 640);
    tensor *c5 = tensor_slice(ctx->scratch, fc, 0, 7, 5), *s5 = tensor_slice(ctx->scratch, fs, 0, 7, 5);
    tensor *c5c = tensor_contiguous(ctx->scratch, c5), *s5c = tensor_contiguous(ctx->scratch, s5);
    tensor_rope(ctx->scratch, xr, c5c, s5c);
    j_floats("op_rope_y", xrd, 640);

    /* swiglu over a wide range */
    int n = 1000;
    tensor *gg = tensor_zeros(ctx->data, 1, (int[]){n}, 0), *uu = tensor_zeros(ctx->data, 1, (int[]){n}, 0);
    float *ggd = tensor_data_ptr(gg), *uud = tensor_data_ptr(uu);
    for (int i = 0; i < n; i++) { ggd[i] = dnn_rng_normal(&r) * 6.0f; uud[i] = dnn_rng_normal(&r); }
    tensor *sw = tensor_swiglu(ctx->scratch, gg, uu);
    j_floats("op_swiglu_g", ggd, n); j_floats("op_swiglu_u", uud, n); j_floats("op_swiglu_y", tensor_data_ptr(sw), n);
    dnn_no_grad_exit(g);
    mem_pool_reset(ctx->scratch);
}

int main(int argc, char **argv) {
    int quick = (argc > 1 && strcmp(argv[1], "quick") == 0);
    char path[512]; snprintf(path, sizeof path, "%s/index.json", OUT);
    J = fopen(path, "w");
    if (!J) { perror(path); return 1; }
    fputc('{', J);

    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, (size_t)1600 << 20, (size_t)512 << 20, (size_t)512 << 20)) return 1;

    gen_rng();
    gen_ops(&ctx);

    /* ---- C1: tiny (V=128 D=256 L=4 H=4 F=683), seed 1, prompt seed 101, P=16, 240 new */
    {
        double t0 = now();
        decoder_lm *lm = make_model(&ctx, 1, 128, 256, 4, 4, 683, 256, 0.02f);
        params_hash("c1_params", lm);
        int P = 16, NEW = 240, prompt[16];
        prompt_ids(101, 128, P, prompt);
        j_ints("c1_prompt", prompt, P);
        int *out = malloc(sizeof(int) * (P + NEW));
        float *lg = malloc(sizeof(float) * (size_t)(NEW + 1) * 128);
        float *mg = malloc(sizeof(float) * (NEW + 1));
        int n = manual_generate(&ctx, lm, prompt, P, NEW, out, lg, mg, NULL, NULL);
        j_ints("c1_tokens", out, n);
        j_floats("c1_margins", mg, n - P);
        bin("c1_logits.f32", lg, sizeof(float) * (size_t)(n - P) * 128);
        /* the library's own generate must agree with the loop above */
        tensor *pt = tensor_zeros_data(ctx.data, 2, (int[]){1, P});
        memcpy(pt->data, prompt, sizeof(int) * P);
        int n2; int *o2 = decoder_lm_generate(ctx.scratch, ctx.data, lm, pt, NEW, 0.0f, 1, &n2);
        j_ints("c1_generate_tokens", o2, n2);
        /* no-cache generate on a short run (gpt.c:381-414) */
        int n3; int *o3 = decoder_lm_generate(ctx.scratch, ctx.data, lm, pt, 24, 0.0f, 0, &n3);
        j_ints("c1_nocache_tokens", o3, n3);
        /* decoder_lm_forward logits over the first 24 tokens of the run */
        tensor *ids = tensor_zeros_data(ctx.data, 2, (int[]){1, 24});
        memcpy(ids->data, out, sizeof(int) * 24);
        dnn_grad_ctx g = dnn_no_grad_enter();
        tensor *fl = decoder_lm_forward(ctx.scratch, lm, ids);
        bin("c1_full24_logits.f32", tensor_data_ptr(fl), sizeof(float) * 24 * 128);
        dnn_no_grad_exit(g);
        mem_pool_reset(ctx.scratch);

        /* multi-token cached prefill of the prompt (one call per layer with N_new=P),
         * then 8 single-token steps; logits of the last prefill row + each step */
        {
            size_t mark = mem_pool_mark(ctx.data);
            kv_cache *c[4];
            for (int i = 0; i < 4; i++) c[i] = kv_cache_create(ctx.data, 1, 4, 64, 64);
            dnn_grad_ctx g2 = dnn_no_grad_enter();
            tensor *idp = tensor_zeros_data(ctx.data, 2, (int[]){1, P});
            memcpy(idp->data, prompt, sizeof(int) * P);
            tensor *h = decoder_lm_token_embeds(ctx.scratch, lm, idp);
            for (int i = 0; i < 4; i++) h = transformer_block_forward_cached(ctx.scratch, lm->blocks[i], h, c[i]);
            h = rms_norm_forward(ctx.scratch, lm->norm, h);
            tensor *l = decoder_lm_lm_head_forward(ctx.scratch, lm, h);
            float pre[9 * 128];
            memcpy(pre, (float*)tensor_data_ptr(l) + (P - 1) * 128, 128 * 4);
            int id = decoder_lm_argmax_token(pre, 128);
            int seq[9]; seq[0] = id;
            mem_pool_reset(ctx.scratch);
            tensor *one = tensor_zeros_data(ctx.data, 1, (int[]){1});
            for (int s = 1; s < 9; s++) {
                ((int*)one->data)[0] = id;
                tensor *e = embedding_forward(ctx.scratch, NULL, lm->embed, one);
                tensor *hh = tensor_reshape(ctx.scratch, e, 3, (int[]){1, 1, 256});
                for (int i = 0; i < 4; i++) hh = transformer_block_forward_cached(ctx.scratch, lm->blocks[i], hh, c[i]);
                hh = rms_norm_forward(ctx.scratch, lm->norm, hh);
                tensor *ll = decoder_lm_lm_head_forward(ctx.scratch, lm, hh);
                memcpy(pre + s * 128, tensor_data_ptr(ll), 128 * 4);
                id = decoder_lm_argmax_token(pre + s * 128, 128);
                seq[s] = id;
                mem_pool_reset(ctx.scratch);
            }
            dnn_no_grad_exit(g2);
            bin("c1_prefill_logits.f32", pre, sizeof pre);
            j_ints("c1_prefill_tokens", seq, 9);
            mem_pool_release(ctx.data, mark);
        }

        /* batch rows: 6 independent B=1 runs, prompt lengths 4..16 (stream 301) */
        {
            dnn_rng r = dnn_rng_seed(301);
            int lens[6], all[6 * 16], toks[6 * (16 + 32)];
            for (int b = 0; b < 6; b++) {
                lens[b] = 4 + dnn_rng_uniform_int(&r, 13);
                for (int i = 0; i < 16; i++) all[b * 16 + i] = dnn_rng_uniform_int(&r, 128);
            }
            for (int b = 0; b < 6; b++) {
                int o[16 + 32];
                int nn = manual_generate(&ctx, lm, all + b * 16, lens[b], 32, o, NULL, NULL, NULL, NULL);
                for (int i = 0; i < 16 + 32; i++) toks[b * 48 + i] = i < nn ? o[i] : -1;
            }
            j_ints("c1_batch_lens", lens, 6);
            j_ints("c1_batch_prompts", all, 6 * 16);
            j_ints("c1_batch_tokens", toks, 6 * 48);
        }
        j_num("c1_seconds", now() - t0);
        free(out); free(lg); free(mg);
        mem_pool_reset(ctx.params); mem_pool_reset(ctx.data);
    }

    /* ---- gpt2-style init (decoder_lm_init_weights) hash on the C1 shape, seed 7 */
    {
        dnn_seed(7);
        decoder_lm *lm = decoder_lm_create(ctx.params, 128, 256, 4, 4, 64, 683);
        params_hash("c1_create_params", lm);
        decoder_lm_init_weights(lm);
        params_hash("c1_gpt2_params", lm);
        mem_pool_reset(ctx.params);
    }

    /* ---- prefix-LM (VLM-shaped, tiny): I=12 bidirectional rows of N(0,1) embeds,
     * then 4 text tokens, one cached_ex(PREFIX_LM) pass, then 6 decode steps.
     * V=96, D=128, L=2, H=2, F=256, seed 5; embeds from stream 505. */
    {
        decoder_lm *lm = make_model(&ctx, 5, 96, 128, 2, 2, 256, 64, 0.02f);
        params_hash("vlm_params", lm);
        int I = 12, T = 4, NS = 6;
        float *emb = malloc(sizeof(float) * I * 128);
        dnn_rng r = dnn_rng_seed(505);
        for (int i = 0; i < I * 128; i++) emb[i] = dnn_rng_normal(&r);
        int txt[4];
        for (int i = 0; i < T; i++) txt[i] = dnn_rng_uniform_int(&r, 96);
        j_floats("vlm_prefix", emb, I * 128);
        j_ints("vlm_text", txt, T);
        size_t mark = mem_pool_mark(ctx.data);
        kv_cache *c[2];
        for (int i = 0; i < 2; i++) c[i] = kv_cache_create(ctx.data, 1, 2, I + T + NS, 64);
        dnn_grad_ctx g = dnn_no_grad_enter();
        tensor *img = tensor_zeros(ctx.data, 3, (int[]){1, I, 128}, 0);
        memcpy(tensor_data_ptr(img), emb, sizeof(float) * I * 128);
        tensor *tid = tensor_zeros_data(ctx.data, 2, (int[]){1, T});
        memcpy(tid->data, txt, sizeof txt);
        tensor *te = decoder_lm_token_embeds(ctx.scratch, lm, tid);
        tensor *h = tensor_cat(ctx.scratch, img, te, 1);
        for (int i = 0; i < 2; i++) h = transformer_block_forward_cached_ex(ctx.scratch, lm->blocks[i], h, c[i], ATTENTION_PREFIX_LM, I);
        h = rms_norm_forward(ctx.scratch, lm->norm, h);
        tensor *l = decoder_lm_lm_head_forward(ctx.scratch, lm, h);
        float *all = malloc(sizeof(float) * (I + T + NS) * 96);
        memcpy(all, tensor_data_ptr(l), sizeof(float) * (I + T) * 96);
        int id = decoder_lm_argmax_token(all + (I + T - 1) * 96, 96);
        int seq[7]; seq[0] = id;
        mem_pool_reset(ctx.scratch);
        tensor *one = tensor_zeros_data(ctx.data, 1, (int[]){1});
        for (int s = 1; s <= NS; s++) {
            ((int*)one->data)[0] = id;
            tensor *e = embedding_forward(ctx.scratch, NULL, lm->embed, one);
            tensor *hh = tensor_reshape(ctx.scratch, e, 3, (int[]){1, 1, 128});
            for (int i = 0; i < 2; i++) hh = transformer_block_forward_cached(ctx.scratch, lm->blocks[i], hh, c[i]);
            hh = rms_norm_forward(ctx.scratch, lm->norm, hh);
            tensor *ll = decoder_lm_lm_head_forward(ctx.scratch, lm, hh);
            memcpy(all + (I + T + s - 1) * 96, tensor_data_ptr(ll), 96 * 4);
            id = decoder_lm_argmax_token(all + (I + T + s - 1) * 96, 96);
            seq[s] = id;
            mem_pool_reset(ctx.scratch);
        }
        dnn_no_grad_exit(g);
        bin("vlm_logits.f32", all, sizeof(float) * (I + T + NS) * 96);
        j_ints("vlm_tokens", seq, NS + 1);
        mem_pool_release(ctx.data, mark);
        free(emb); free(all);
        mem_pool_reset(ctx.params); mem_pool_reset(ctx.data);
    }

    /* ---- C1 shape, GPT-2 init: seed 11, prompt seed 111, P=16, 240 new */
    {
        decoder_lm *lm = make_model_gpt2(&ctx, 11, 128, 256, 4, 4, 683, 256);
        params_hash("c1g_params", lm);
        int P = 16, NEW = 240, prompt[16];
        prompt_ids(111, 128, P, prompt);
        j_ints("c1g_prompt", prompt, P);
        int *out = malloc(sizeof(int) * (P + NEW));
        float *lg = malloc(sizeof(float) * (size_t)(NEW + 1) * 128);
        float *mg = malloc(sizeof(float) * (NEW + 1));
        int n = manual_generate(&ctx, lm, prompt, P, NEW, out, lg, mg, NULL, NULL);
        j_ints("c1g_tokens", out, n);
        j_floats("c1g_margins", mg, n - P);
        bin("c1g_logits.f32", lg, sizeof(float) * (size_t)(n - P) * 128);
        free(out); free(lg); free(mg);
        mem_pool_reset(ctx.params); mem_pool_reset(ctx.data);
    }

    /* ---- C2 shape, GPT-2 init: seed 12, prompt seed 112, P=32, 128 new */
    {
        int NEW = quick ? 8 : 128;
        decoder_lm *lm = make_model_gpt2(&ctx, 12, 8192, 768, 12, 12, 2048, 1088);
        params_hash("c2g_params", lm);
        int P = 32, prompt[32];
        prompt_ids(112, 8192, P, prompt);
        j_ints("c2g_prompt", prompt, P);
        int *out = malloc(sizeof(int) * (P + NEW));
        float *mg = malloc(sizeof(float) * (NEW + 1));
        uint64_t *hs = malloc(sizeof(uint64_t) * (NEW + 1));
        float *f8 = malloc(sizeof(float) * 8 * (NEW + 1));
        int n = manual_generate(&ctx, lm, prompt, P, NEW, out, NULL, mg, hs, f8);
        j_ints("c2g_tokens", out, n);
        j_floats("c2g_margins", mg, n - P);
        j_floats("c2g_first8", f8, 8 * (n - P));
        key("c2g_logit_hashes"); fputc('[', J);
        for (int i = 0; i < n - P; i++) fprintf(J, "%s\"%016llx\"", i ? "," : "", (unsigned long long)hs[i]);
        fputc(']', J);
        free(out); free(mg); free(hs); free(f8);
        mem_pool_reset(ctx.params); mem_pool_reset(ctx.data);
    }

    /* ---- C2: medium (V=8192 D=768 L=12 H=12 F=2048), seed 2, prompt seed 102, P=32 */
    {
        double t0 = now();
        int NEW = quick ? 16 : 512;
        decoder_lm *lm = make_model(&ctx, 2, 8192, 768, 12, 12, 2048, 1088, 0.02f);
        params_hash("c2_params", lm);
        int P = 32, prompt[32];
        prompt_ids(102, 8192, P, prompt);
        j_ints("c2_prompt", prompt, P);
        int *out = malloc(sizeof(int) * (P + NEW));
        float *mg = malloc(sizeof(float) * (NEW + 1));
        uint64_t *hs = malloc(sizeof(uint64_t) * (NEW + 1));
        float *f8 = malloc(sizeof(float) * 8 * (NEW + 1));
        float *lg = malloc(sizeof(float) * 4 * 8192);
        int n = manual_generate(&ctx, lm, prompt, P, NEW, out, NULL, mg, hs, f8);
        j_ints("c2_tokens", out, n);
        j_floats("c2_margins", mg, n - P);
        j_floats("c2_first8", f8, 8 * (n - P));
        key("c2_logit_hashes"); fputc('[', J);
        for (int i = 0; i < n - P; i++) fprintf(J, "%s\"%016llx\"", i ? "," : "", (unsigned long long)hs[i]);
        fputc(']', J);
        /* full logits of the first 4 generated steps */
        manual_generate(&ctx, lm, prompt, P, 4, out, lg, NULL, NULL, NULL);
        bin("c2_logits4.f32", lg, sizeof(float) * 4 * 8192);
        j_num("c2_seconds", now() - t0);
        j_num("c2_new", NEW);
    }

    fputs("\n}\n", J);
    fclose(J);
    dnn_ctx_destroy(&ctx);
    return 0;
}
