/* gpt.c -- decoder LM construction, initialisation and generation.
 *
 * Construction and init follow the reference (src/gpt.c:16-62, 431-496) so the
 * same seed gives the same parameters.  Generation (src/gpt.c:258-421) runs on
 * the MI355X: the whole token loop -- prompt tokens one at a time, then greedy
 * steps -- is one persistent kernel launch (dnn_hip_generate).  With
 * temperature > 0 each step's logits come back to the host and are sampled with
 * the reference's sampler and thread-local RNG.  use_cache=0 asks the reference
 * to recompute the prefix every step; that recomputation yields the same
 * logits row by row (each row's GEMV, norm and attention sums are the same
 * float sequences), so both modes take the cached device path here. */
#include "dnn/gpt.h"
#include "dnn/rng.h"
#include "dnn/rope.h"
#include "dnn/autograd.h"
#include "dnn/tokenizer.h"
#include "dnn_hip.h"
#include "device.h"
#include <assert.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

decoder_lm *decoder_lm_create(struct mem_pool *params_pool, int vocab_size, int d_model,
                              int n_layers, int n_heads, int d_k, int intermediate_size) {
    assert(vocab_size > 0 && d_model > 0 && n_layers > 0);
    assert(n_heads > 0 && d_k > 0 && intermediate_size > 0);
    assert(d_model == n_heads * d_k && "d_model must equal n_heads * d_k");
    decoder_lm *lm = _mem_pool_alloc(params_pool, sizeof(decoder_lm), NULL);
    module_init(&lm->base, params_pool, "decoder_lm");
    lm->d_model = d_model;
    lm->vocab_size = vocab_size;
    lm->n_layers = n_layers;
    lm->embed = embedding_create(params_pool, vocab_size, d_model);
    module_add_child(&lm->base, "embed", &lm->embed->base);
    lm->blocks = _mem_pool_alloc(params_pool, sizeof(transformer_block *) * (size_t)n_layers, NULL);
    for (int i = 0; i < n_layers; i++) {
        lm->blocks[i] = transformer_block_create(params_pool, d_model, n_heads, d_k, intermediate_size);
        char buf[32];
        int len = snprintf(buf, sizeof buf, "blocks.%d", i);
        char *name = _mem_pool_alloc(params_pool, (size_t)len + 1, buf);
        module_add_child(&lm->base, name, &lm->blocks[i]->base);
    }
    lm->norm = rms_norm_create(params_pool, d_model, 1e-5f);
    module_add_child(&lm->base, "norm", &lm->norm->base);
    /* tied lm_head: no weight of its own, a zero bias [V] */
    lm->lm_head = _mem_pool_alloc(params_pool, sizeof(linear), NULL);
    module_init(&lm->lm_head->base, params_pool, "linear");
    lm->lm_head->in_features = d_model;
    lm->lm_head->out_features = vocab_size;
    lm->lm_head->weight = NULL;
    lm->lm_head->bias = tensor_zeros(params_pool, 1, (int[]){vocab_size}, 1);
    module_param(&lm->lm_head->base, "bias", lm->lm_head->bias);
    module_add_child(&lm->base, "lm_head", &lm->lm_head->base);
    dnn_amd_register_lm(lm);
    return lm;
}

long long decoder_lm_num_parameters(decoder_lm *lm) { return module_num_parameters(&lm->base); }

/* GPT-2 style: N(0, 1/sqrt(D)) for the embedding and every linear weight,
 * residual projections (out_proj, down_proj) scaled by 1/sqrt(2L), biases 0;
 * the module walk visits linears in registration order (gpt.c:431-477). */
static void init_linear(linear *l, float std) {
    if (l->weight) {
        float *w = tensor_data_ptr(l->weight);
        for (int i = 0, n = tensor_numel(l->weight); i < n; i++) w[i] = dnn_rng_normal(dnn_get_rng()) * std;
    }
    memset(tensor_data_ptr(l->bias), 0, sizeof(float) * (size_t)tensor_numel(l->bias));
}

static void init_walk(module *m, float std, float residual_std) {
    for (module_item *it = m->items_head; it; it = it->next) {
        if (it->kind != MODULE_ITEM_CHILD) continue;
        module *c = it->as.child;
        if (strcmp(c->type_name, "linear") == 0)
            init_linear((linear *)c, (strstr(it->name, "out_proj") || strstr(it->name, "down_proj")) ? residual_std : std);
        else
            init_walk(c, std, residual_std);
    }
}

void decoder_lm_init_weights(decoder_lm *lm) {
    assert(lm);
    const float std = 1.0f / sqrtf((float)lm->d_model);
    const float residual_std = std / sqrtf(2.0f * (float)lm->n_layers);
    float *e = tensor_data_ptr(lm->embed->weight);
    for (int i = 0, n = tensor_numel(lm->embed->weight); i < n; i++) e[i] = dnn_rng_normal(dnn_get_rng()) * std;
    init_walk(&lm->base, std, residual_std);
}

void decoder_lm_init_normal(decoder_lm *lm, float std) {
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    for (int i = 0; i < n; i++) {
        int gamma = ps[i] == lm->norm->weight;
        for (int l = 0; l < lm->n_layers; l++)
            gamma |= ps[i] == lm->blocks[l]->attn_norm->weight || ps[i] == lm->blocks[l]->ffn_norm->weight;
        if (gamma) continue;
        float *d = tensor_data_ptr(ps[i]);
        for (int j = 0, ne = tensor_numel(ps[i]); j < ne; j++) d[j] = dnn_rng_normal(dnn_get_rng()) * std;
    }
}

void decoder_lm_enable_rope(struct mem_pool *params_pool, decoder_lm *lm, int max_seq_len, float base) {
    assert(lm && max_seq_len > 0);
    const int d_k = lm->blocks[0]->d_k;
    assert(d_k % 2 == 0 && "RoPE requires even head dimension");
    tensor *c, *s;
    tensor_rope_freqs_init(params_pool, &c, &s, d_k, max_seq_len, base);
    for (int i = 0; i < lm->n_layers; i++) {
        lm->blocks[i]->freqs_cos = c;
        lm->blocks[i]->freqs_sin = s;
    }
}

/* first index of the maximum (gpt.c:220-230) */
int decoder_lm_argmax_token(const float *logits, int vocab_size) {
    int best = 0;
    for (int i = 1; i < vocab_size; i++)
        if (logits[i] > logits[best]) best = i;
    return best;
}

/* softmax(logits / temp) sampled by inverse CDF with one uniform draw from the
 * default stream (gpt.c:232-254); the running sum adds each probability in
 * index order, so the chosen index matches the reference for the same logits. */
int decoder_lm_sample_with_temp(const float *logits, int vocab_size, float temp) {
    const float inv = 1.0f / temp;
    float mx = -INFINITY;
    for (int i = 0; i < vocab_size; i++) { float v = logits[i] * inv; if (v > mx) mx = v; }
    float sum = 0.0f;
    for (int i = 0; i < vocab_size; i++) sum += expf(logits[i] * inv - mx);
    const float r = dnn_rng_uniform(dnn_get_rng());
    float cum = 0.0f;
    for (int i = 0; i < vocab_size; i++) {
        cum += expf(logits[i] * inv - mx) / sum;
        if (r < cum) return i;
    }
    return vocab_size - 1;
}

int *decoder_lm_generate(struct mem_pool *scratch_pool, struct mem_pool *data_pool, decoder_lm *lm,
                         const tensor *prompt_ids, int max_new_tokens, float temperature, int use_cache,
                         int *n_out) {
    (void)scratch_pool;
    (void)use_cache;
    assert(lm && prompt_ids);
    assert(prompt_ids->ndim == 2 && "generate: prompt_ids must be 2D [1, N]");
    assert(prompt_ids->shape[0] == 1 && "generate: only batch=1 supported");
    assert(prompt_ids->contiguous && "generate: prompt_ids must be contiguous");
    assert(max_new_tokens > 0);
    assert(temperature >= 0.0f && "generate: temperature must be >= 0");
    const int P = prompt_ids->shape[1], max_len = P + max_new_tokens, V = lm->vocab_size;
    int *out = _mem_pool_alloc(data_pool, sizeof(int) * (size_t)max_len, NULL);
    memcpy(out, (const int *)prompt_ids->data + prompt_ids->offset, sizeof(int) * (size_t)P);
    for (int i = 0; i < P; i++) assert(out[i] >= 0 && out[i] < V && "embedding: id out of range");
    dnn_grad_ctx g = dnn_no_grad_enter();
    dnn_hip_model *dm = dnn_amd_device_model(lm);
    int n = P;
    if (temperature == 0.0f) {
        int rc = dnn_hip_generate(dm, out, P, max_new_tokens, TOKENIZER_EOS_ID, out, &n);
        dnn_amd_check(rc, "dnn_hip_generate");
    } else {
        dnn_hip_session *s = NULL;
        dnn_amd_check(dnn_hip_session_create(dm, 1, max_len, &s), "dnn_hip_session_create");
        float *lg = malloc(sizeof(float) * (size_t)P * V);
        int *ids = malloc(sizeof(int) * (size_t)P);
        assert(lg && ids);
        /* prompt: P steps, keep the last row of logits */
        dnn_amd_check(dnn_hip_decode(s, out, P, NULL, P, -1, ids, lg, NULL), "dnn_hip_decode");
        int id = decoder_lm_sample_with_temp(lg + (size_t)(P - 1) * V, V, temperature);
        out[n++] = id;
        while (id != TOKENIZER_EOS_ID && n < max_len) {
            dnn_amd_check(dnn_hip_decode(s, &id, 1, NULL, 1, -1, ids, lg, NULL), "dnn_hip_decode");
            id = decoder_lm_sample_with_temp(lg, V, temperature);
            out[n++] = id;
        }
        free(lg);
        free(ids);
        dnn_hip_session_destroy(s);
    }
    dnn_no_grad_exit(g);
    *n_out = n;
    return out;
}
