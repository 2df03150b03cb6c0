/*
 * gen_sample.c -- writes tests/golden/data/sample.json: the ids the REAL
 * reference's decoder_lm_generate(temperature > 0, use_cache = 1) draws for a
 * seed (gpt.c:232-254 sampling, rng.c default stream), plus, per generated
 * token, how far the uniform draw r sat from the nearest edge of the chosen
 * token's CDF interval.  Dev container only (links oracle/_ref/libdnnref.so);
 * the JSON is committed data.  Build + run: tests/golden/make_golden.sh.
 *
 * The margin of a step is min(r - cum_lo, cum_hi - r) over the running sum the
 * reference's sampler forms: a device whose logits differ from the reference's
 * in the last bits can draw another token only at a step whose margin is of
 * the order of those differences.  The margins come from the same cached
 * forward the reference's generate runs (transformer_block_forward_cached per
 * token), replayed from the same RNG state, and the replay's ids are checked
 * against decoder_lm_generate's own.
 */
#include "dnn.h"
#include "gpt.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static FILE *J;

/* the reference sampler's running sum (gpt.c:232-254), reporting the draw's
 * distance to the chosen interval's edges; consumes the same one draw */
static int sample_margin(const float *logits, int V, float temp, double *margin) {
    const float inv = 1.0f / temp;
    float mx = -INFINITY;
    for (int i = 0; i < V; i++) { float v = logits[i] * inv; if (v > mx) mx = v; }
    float sum = 0.0f;
    for (int i = 0; i < V; i++) sum += expf(logits[i] * inv - mx);
    const float r = dnn_rng_uniform(dnn_get_rng());
    float cum = 0.0f, prev = 0.0f;
    for (int i = 0; i < V; i++) {
        prev = cum;
        cum += expf(logits[i] * inv - mx) / sum;
        if (r < cum) {
            const double a = (double)r - prev, b = (double)cum - r;
            *margin = a < b ? a : b;
            return i;
        }
    }
    *margin = 0.0;
    return V - 1;
}

static void run(const char *name, int V, int D, int L, int H, int F, unsigned long long seed,
                unsigned long long pseed, int P, int NEW, float temp, int first) {
    dnn_ctx ctx;
    size_t need = (size_t)(V * D + L * (4 * D * D + 3 * D * F + 8 * D + 2 * F) + 4 * V) * 4 + ((size_t)64 << 20);
    if (dnn_ctx_init(&ctx, need, (size_t)256 << 20, (size_t)512 << 20)) exit(1);
    dnn_seed(seed);
    decoder_lm *lm = decoder_lm_create(ctx.params, V, D, L, H, D / H, F);
    decoder_lm_init_weights(lm);
    decoder_lm_enable_rope(ctx.params, lm, P + NEW, 10000.0f);
    dnn_rng r = dnn_rng_seed(pseed);
    tensor *prompt = tensor_zeros_data(ctx.data, 2, (int[]){1, P});
    for (int i = 0; i < P; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, V);
    const dnn_rng saved = *dnn_get_rng();

    int n_out = 0;
    int *out = decoder_lm_generate(ctx.scratch, ctx.data, lm, prompt, NEW, temp, 1, &n_out);

    /* replay: the cached forward of generate, from the same RNG state */
    *dnn_get_rng() = saved;
    dnn_grad_ctx g = dnn_no_grad_enter();
    kv_cache **caches = malloc(sizeof(kv_cache *) * (size_t)L);
    for (int l = 0; l < L; l++) caches[l] = kv_cache_create(ctx.data, 1, H, P + NEW, D / H);
    int *ids = malloc(sizeof(int) * (size_t)(P + NEW));
    double *marg = malloc(sizeof(double) * (size_t)NEW);
    memcpy(ids, prompt->data, sizeof(int) * (size_t)P);
    tensor *one = tensor_zeros_data(ctx.data, 1, (int[]){1});
    int n = P, k = 0;
    for (int t = 0; n < P + NEW; t++) {
        ((int *)one->data)[0] = ids[t];
        tensor *e = embedding_forward(ctx.scratch, NULL, lm->embed, one);
        tensor *h = tensor_reshape(ctx.scratch, e, 3, (int[]){1, 1, D});
        for (int l = 0; l < L; l++) h = transformer_block_forward_cached(ctx.scratch, lm->blocks[l], h, caches[l]);
        if (t >= P - 1) {
            h = rms_norm_forward(ctx.scratch, lm->norm, h);
            tensor *lg = decoder_lm_lm_head_forward(ctx.scratch, lm, h);
            ids[n++] = sample_margin(tensor_data_ptr(lg), V, temp, &marg[k++]);
            if (ids[n - 1] == TOKENIZER_EOS_ID) break;
        }
        mem_pool_reset(ctx.scratch);
    }
    dnn_no_grad_exit(g);
    if (n != n_out || memcmp(ids, out, sizeof(int) * (size_t)n) != 0) {
        fprintf(stderr, "%s: the replay drew other ids than decoder_lm_generate\n", name);
        exit(1);
    }
    fprintf(J, "%s\"%s\": {\"V\": %d, \"D\": %d, \"L\": %d, \"H\": %d, \"F\": %d, \"seed\": %llu, \"prompt_seed\": %llu, "
               "\"P\": %d, \"new\": %d, \"temp\": %.9g, \"tokens\": [", first ? "" : ",\n", name, V, D, L, H, F, seed,
            pseed, P, NEW, temp);
    for (int i = 0; i < n_out; i++) fprintf(J, "%s%d", i ? "," : "", out[i]);
    fprintf(J, "], \"margins\": [");
    for (int i = 0; i < k; i++) fprintf(J, "%s%.9g", i ? "," : "", marg[i]);
    fprintf(J, "]}");
    free(caches); free(ids); free(marg);
    dnn_ctx_destroy(&ctx);
}

int main(void) {
    J = fopen("tests/golden/data/sample.json", "w");
    if (!J) return 1;
    fprintf(J, "{\n");
    run("c1g_t08", 128, 256, 4, 4, 683, 11, 111, 16, 64, 0.8f, 1);
    run("c1g_t15", 128, 256, 4, 4, 683, 11, 111, 16, 64, 1.5f, 0);
    run("c2g_t10", 8192, 768, 12, 12, 2048, 12, 112, 32, 48, 1.0f, 0);
    fprintf(J, "\n}\n");
    fclose(J);
    return 0;
}
