/* blocks.c -- the reference's layer-level forward API on the device:
 * transformer_block_forward_cached(_ex) (transformer.c:211-426),
 * rms_norm_forward (nn.c:169-173), decoder_lm_lm_head_forward (gpt.c:117-122),
 * decoder_lm_token_embeds / forward_embeds(_ex) / forward (gpt.c:66-151) and
 * kv_cache_get_K/V (transformer.c:90-112) for caches the device path holds.
 *
 * A transformer_block is found in the decoder_lm it belongs to (every model
 * built by decoder_lm_create is registered), so a block call runs that model's
 * layer on its HBM mirror.  The reference keeps one kv_cache per layer; here
 * the first call that uses a cache binds it to layer `l` of a device session
 * (K/V in HBM, [layer][row][head] as the decode kernels read them).  Caches of
 * the same model, batch and length share one session, one layer slot each.
 * The cache struct's seq_len stays the source of truth for positions;
 * kv_cache_get_K/V copy the device rows back into the cache's host tensors. */
#include "dnn/transformer.h"
#include "dnn/gpt.h"
#include "dnn_hip.h"
#include "device.h"
#include <assert.h>
#include <stdlib.h>
#include <string.h>

#define MAX_MODELS 64
#define MAX_GROUPS 64
#define MAX_LAYERS 64

static decoder_lm *g_models[MAX_MODELS];

typedef struct {
    decoder_lm *lm;
    int B, max_seq;
    dnn_hip_session *s;
    kv_cache *slot[MAX_LAYERS];
} cache_group;

static cache_group g_groups[MAX_GROUPS];

void dnn_amd_register_lm(decoder_lm *lm) {
    for (int i = 0; i < MAX_MODELS; i++)
        if (g_models[i] == lm) return;
    for (int i = 0; i < MAX_MODELS; i++)
        if (!g_models[i]) { g_models[i] = lm; return; }
    assert(0 && "dnn_amd: too many decoder_lm models");
}

static decoder_lm *model_of_block(transformer_block *blk, int *layer) {
    for (int i = 0; i < MAX_MODELS; i++) {
        decoder_lm *lm = g_models[i];
        if (!lm) continue;
        for (int l = 0; l < lm->n_layers; l++)
            if (lm->blocks[l] == blk) { *layer = l; return lm; }
    }
    return NULL;
}

static void unbind(cache_group *cg, int l) {
    cg->slot[l] = NULL;
    for (int i = 0; i < MAX_LAYERS; i++)
        if (cg->slot[i]) return;
    dnn_hip_session_destroy(cg->s);
    memset(cg, 0, sizeof *cg);
}

/* The session and layer slot a cache is bound to (binding it on first use).
 * Caches live in the caller's pools, so a released cache's address can come
 * back for a new one: a binding whose batch or length no longer matches the
 * struct at that address is dropped and the cache bound afresh. */
static dnn_hip_session *session_of_cache(kv_cache *c, decoder_lm *lm, int layer, int bind) {
    const int B = c->k_cache->shape[0];
    for (int g = 0; g < MAX_GROUPS; g++)
        for (int l = 0; g_groups[g].s && l < MAX_LAYERS; l++)
            if (g_groups[g].slot[l] == c) {
                cache_group *cg = &g_groups[g];
                if (cg->B == B && cg->max_seq == c->max_seq && (!lm || cg->lm == lm)) {
                    assert((layer < 0 || l == layer) && "kv_cache used with two different layers");
                    return cg->s;
                }
                unbind(cg, l);
                g = MAX_GROUPS;
                break;
            }
    if (!bind) return NULL;
    assert(layer >= 0 && layer < MAX_LAYERS);
    for (int g = 0; g < MAX_GROUPS; g++) {
        cache_group *cg = &g_groups[g];
        if (cg->s && cg->lm == lm && cg->B == B && cg->max_seq == c->max_seq && !cg->slot[layer]) {
            cg->slot[layer] = c;
            return cg->s;
        }
    }
    for (int g = 0; g < MAX_GROUPS; g++) {
        cache_group *cg = &g_groups[g];
        if (cg->s) continue;
        dnn_amd_check(dnn_hip_session_create(dnn_amd_device_model(lm), B, c->max_seq, &cg->s),
                      "dnn_hip_session_create");
        cg->lm = lm;
        cg->B = B;
        cg->max_seq = c->max_seq;
        memset(cg->slot, 0, sizeof cg->slot);
        cg->slot[layer] = c;
        return cg->s;
    }
    assert(0 && "dnn_amd: too many device-bound kv caches");
    return NULL;
}

static int layer_of_cache(kv_cache *c) {
    for (int g = 0; g < MAX_GROUPS; g++)
        for (int l = 0; g_groups[g].s && l < MAX_LAYERS; l++)
            if (g_groups[g].slot[l] == c)
                return g_groups[g].B == c->k_cache->shape[0] && g_groups[g].max_seq == c->max_seq ? l : -1;
    return -1;
}

int dnn_amd_cache_is_bound(kv_cache *c) { return layer_of_cache(c) >= 0; }

tensor *transformer_block_forward_cached_ex(struct mem_pool *scratch, transformer_block *block, const tensor *x,
                                            kv_cache *cache, attention_mode mode, int prefix_len) {
    assert(block && x && cache);
    assert(x->contiguous && "cached forward: x must be contiguous");
    assert(x->ndim == 3 && "cached forward: x must be [B, N_new, d_model]");
    assert(x->shape[2] == block->d_model);
    if (mode == ATTENTION_PREFIX_LM) assert(cache->seq_len == 0 && "prefix-LM prefill requires empty cache");
    const int B = x->shape[0], N = x->shape[1], D = x->shape[2];
    assert(B == cache->k_cache->shape[0] && block->n_heads == cache->k_cache->shape[1]);
    assert(cache->seq_len + N <= cache->max_seq && "kv_cache: cache full");
    int layer = -1;
    decoder_lm *lm = model_of_block(block, &layer);
    assert(lm && "transformer_block_forward_cached: the block belongs to no decoder_lm (device path)");
    (void)dnn_amd_device_model(lm);                    /* mirror current weights and RoPE table */
    dnn_hip_session *s = session_of_cache(cache, lm, layer, 1);
    tensor *y = tensor_scratch(scratch, 3, (int[]){B, N, D}, 0);
    dnn_amd_check(dnn_hip_block_forward(s, layer, (const float *)x->data + x->offset, N, cache->seq_len, (int)mode,
                                        prefix_len, tensor_data_ptr(y)),
                  "dnn_hip_block_forward");
    cache->seq_len += N;
    return y;
}

tensor *transformer_block_forward_cached(struct mem_pool *scratch, transformer_block *block, const tensor *x,
                                         kv_cache *cache) {
    return transformer_block_forward_cached_ex(scratch, block, x, cache, ATTENTION_CAUSAL, 0);
}

/* Copies the device rows [0, seq_len) of a bound cache into its host tensors. */
void dnn_amd_cache_sync(kv_cache *c) {
    const int layer = layer_of_cache(c);
    if (layer < 0 || c->seq_len == 0) return;
    dnn_hip_session *s = session_of_cache(c, NULL, layer, 0);
    const int B = c->k_cache->shape[0], H = c->k_cache->shape[1], dk = c->k_cache->shape[3], S = c->seq_len;
    float *rows = malloc(sizeof(float) * (size_t)B * H * S * dk);
    assert(rows);
    for (int which = 0; which < 2; which++) {
        tensor *t = which ? c->v_cache : c->k_cache;
        dnn_amd_check(dnn_hip_cache_read(s, layer, which, S, rows), "dnn_hip_cache_read");
        float *d = (float *)t->data + t->offset;
        for (int b = 0; b < B; b++)
            for (int h = 0; h < H; h++)
                memcpy(d + (size_t)b * t->strides[0] + (size_t)h * t->strides[1],
                       rows + (((size_t)b * H + h) * S) * dk, sizeof(float) * (size_t)S * dk);
    }
    free(rows);
}

/* A session for whole-model calls of lm (one row, no cache use). */
static dnn_hip_session *util_session(decoder_lm *lm) {
    static decoder_lm *owner[MAX_MODELS];
    static dnn_hip_session *sess[MAX_MODELS];
    dnn_hip_model *dm = dnn_amd_device_model(lm);
    for (int i = 0; i < MAX_MODELS; i++)
        if (owner[i] == lm) return sess[i];
    for (int i = 0; i < MAX_MODELS; i++)
        if (!owner[i]) {
            dnn_amd_check(dnn_hip_session_create(dm, 1, 1, &sess[i]), "dnn_hip_session_create");
            owner[i] = lm;
            return sess[i];
        }
    assert(0 && "dnn_amd: too many models");
    return NULL;
}

/* h [..., d_model] -> logits [..., V] = h . embed^T + bias (no final norm). */
tensor *decoder_lm_lm_head_forward(struct mem_pool *scratch, decoder_lm *lm, const tensor *h) {
    assert(lm && h && h->contiguous && h->shape[h->ndim - 1] == lm->d_model);
    const int n = tensor_numel(h) / lm->d_model;
    int shape[DNN_MAX_DIMS];
    for (int i = 0; i < h->ndim; i++) shape[i] = h->shape[i];
    shape[h->ndim - 1] = lm->vocab_size;
    tensor *out = tensor_scratch(scratch, h->ndim, shape, 0);
    dnn_amd_check(dnn_hip_head_forward(util_session(lm), (const float *)h->data + h->offset, n, 0, tensor_data_ptr(out)),
                  "dnn_hip_head_forward");
    return out;
}

/* input_ids [B, N] -> embeddings [B, N, d_model] (gpt.c:66-81). */
tensor *decoder_lm_token_embeds(struct mem_pool *scratch, decoder_lm *lm, const tensor *input_ids) {
    assert(lm && input_ids);
    assert(input_ids->ndim == 2 && "token_embeds: input_ids must be 2D [B, N]");
    assert(input_ids->contiguous && "token_embeds: input_ids must be contiguous");
    const int B = input_ids->shape[0], N = input_ids->shape[1];
    tensor *flat = tensor_flatten(scratch, (tensor *)input_ids);
    tensor *h = embedding_forward(scratch, NULL, lm->embed, flat);
    return tensor_reshape(scratch, h, 3, (int[]){B, N, lm->d_model});
}

/* B rows of N embeddings x [B][N][D] through layers [l0, l1) (full-sequence
 * attention: an empty cache of length N per row) into `hidden` [B][N][D];
 * then, with `final`, the final rms_norm -- into `hidden` (norm_only) or
 * through the tied head into `logits` [B][N][V].  A session of its own,
 * destroyed on return. */
static void forward_rows(decoder_lm *lm, const float *x, int B, int N, int mode, int prefix_len, int l0, int l1,
                         float *hidden, int final, float *logits) {
    const size_t n = (size_t)B * N * lm->d_model;
    dnn_hip_session *s = NULL;
    dnn_amd_check(dnn_hip_session_create(dnn_amd_device_model(lm), B, N, &s), "dnn_hip_session_create");
    float *a = malloc(sizeof(float) * n), *b = malloc(sizeof(float) * n);
    assert(a && b);
    memcpy(a, x, sizeof(float) * n);
    for (int l = l0; l < l1; l++) {
        dnn_amd_check(dnn_hip_block_forward(s, l, a, N, 0, mode, prefix_len, b), "dnn_hip_block_forward");
        float *t = a; a = b; b = t;
    }
    if (final && logits)
        dnn_amd_check(dnn_hip_head_forward(s, a, B * N, 1, logits), "dnn_hip_head_forward");
    else if (final)
        dnn_amd_check(dnn_hip_op_rms_norm(a, B * N, lm->d_model, tensor_data_ptr(lm->norm->weight), lm->norm->eps, a),
                      "dnn_hip_op_rms_norm");
    if (hidden) memcpy(hidden, a, sizeof(float) * n);
    free(a);
    free(b);
    dnn_hip_session_destroy(s);
}

/* The rows of `in` [B][S][D] through layers [l0, l1) (+ the final norm /
 * head), per seq_lens: batch row b runs as a sequence of its first seq_lens[b]
 * rows (keys past it are never visible, attention.c:272,290); the rows after
 * it, which the reference leaves uncomputed, come back zero. */
static void forward_batch(decoder_lm *lm, const float *in, int B, int S, attention_mode mode, int prefix_len,
                          const int *seq_lens, int l0, int l1, float *hidden, int final, float *logits) {
    const int D = lm->d_model, V = lm->vocab_size;
    assert((mode == ATTENTION_CAUSAL || mode == ATTENTION_PREFIX_LM) && "unknown attention mode");
    if (!seq_lens) {
        forward_rows(lm, in, B, S, mode, prefix_len, l0, l1, hidden, final, logits);
        return;
    }
    for (int b = 0; b < B; b++) {
        const int n = seq_lens[b];
        assert(n >= 0 && n <= S && "seq_lens out of range");
        float *hb = hidden ? hidden + (size_t)b * S * D : NULL;
        float *lb = logits ? logits + (size_t)b * S * V : NULL;
        if (n > 0) forward_rows(lm, in + (size_t)b * S * D, 1, n, mode, prefix_len, l0, l1, hb, final, lb);
        if (hb) memset(hb + (size_t)n * D, 0, sizeof(float) * (size_t)(S - n) * D);
        if (lb) memset(lb + (size_t)n * V, 0, sizeof(float) * (size_t)(S - n) * V);
    }
}

/* embeds [B, S, D] -> logits [B, S, V] (gpt.c:84-144): blocks with full-sequence
 * attention (attention.c:259-380 masks), final rms_norm, tied lm_head. */
tensor *decoder_lm_forward_embeds_ex(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds,
                                     attention_mode mode, int prefix_len, const int *seq_lens) {
    assert(lm && embeds);
    assert(embeds->ndim == 3 && "hidden_from_embeds: embeds must be 3D [B, S, D]");
    assert(embeds->shape[2] == lm->d_model && embeds->contiguous);
    const int B = embeds->shape[0], S = embeds->shape[1], V = lm->vocab_size;
    tensor *logits = tensor_scratch(scratch, 3, (int[]){B, S, V}, 0);
    forward_batch(lm, (const float *)embeds->data + embeds->offset, B, S, mode, prefix_len, seq_lens, 0,
                  lm->n_layers, NULL, 1, tensor_data_ptr(logits));
    return logits;
}

tensor *decoder_lm_forward_embeds(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds) {
    return decoder_lm_forward_embeds_ex(scratch, lm, embeds, ATTENTION_CAUSAL, 0, NULL);
}

/* embeds [B, S, D] -> the final normalised hidden state [B, S, D] (gpt.c:84-113). */
tensor *decoder_lm_hidden_from_embeds_ex(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds,
                                         attention_mode mode, int prefix_len, const int *seq_lens) {
    assert(lm && embeds);
    assert(embeds->ndim == 3 && "hidden_from_embeds: embeds must be 3D [B, S, D]");
    assert(embeds->shape[2] == lm->d_model && embeds->contiguous);
    const int B = embeds->shape[0], S = embeds->shape[1], D = lm->d_model;
    tensor *h = tensor_scratch(scratch, 3, (int[]){B, S, D}, 0);
    forward_batch(lm, (const float *)embeds->data + embeds->offset, B, S, mode, prefix_len, seq_lens, 0, lm->n_layers,
                  tensor_data_ptr(h), 1, NULL);
    return h;
}

tensor *decoder_lm_hidden_from_embeds(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds) {
    return decoder_lm_hidden_from_embeds_ex(scratch, lm, embeds, ATTENTION_CAUSAL, 0, NULL);
}

/* Full-sequence forward of one block (transformer.c:151-208), no cache. */
tensor *transformer_block_forward_ex(struct mem_pool *scratch, transformer_block *block, const tensor *x,
                                     attention_mode mode, int prefix_len, const int *seq_lens) {
    assert(block && x);
    assert(x->ndim == 3 && x->contiguous && "transformer_block_forward: x must be contiguous [B, N, d_model]");
    assert(x->shape[2] == block->d_model);
    int layer = -1;
    decoder_lm *lm = model_of_block(block, &layer);
    assert(lm && "transformer_block_forward: the block belongs to no decoder_lm (device path)");
    const int B = x->shape[0], N = x->shape[1], D = x->shape[2];
    tensor *y = tensor_scratch(scratch, 3, (int[]){B, N, D}, 0);
    forward_batch(lm, (const float *)x->data + x->offset, B, N, mode, prefix_len, seq_lens, layer, layer + 1,
                  tensor_data_ptr(y), 0, NULL);
    return y;
}

tensor *transformer_block_forward(struct mem_pool *scratch, transformer_block *block, const tensor *x) {
    return transformer_block_forward_ex(scratch, block, x, ATTENTION_CAUSAL, 0, NULL);
}

/* input_ids [B, N] -> logits [B, N, V] (gpt.c:148-151). */
tensor *decoder_lm_forward(struct mem_pool *scratch, decoder_lm *lm, const tensor *input_ids) {
    tensor *h = decoder_lm_token_embeds(scratch, lm, input_ids);
    return decoder_lm_forward_embeds(scratch, lm, h);
}
