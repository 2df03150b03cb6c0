/* transformer.c -- KV cache and block construction (reference
 * src/transformer.c:30-147).  The cached forward runs on the device (blocks.c
 * for the per-block API, the decode kernels for generate); a cache it used
 * holds its rows in HBM, and kv_cache_get_K/V copy them back first. */
#include "dnn/transformer.h"
#include "device.h"
#include <assert.h>
#include <string.h>

kv_cache *kv_cache_create(struct mem_pool *params_pool, int B, int H, int max_seq, int d_k) {
    kv_cache *c = _mem_pool_alloc(params_pool, sizeof(kv_cache), NULL);
    const int shape[4] = {B, H, max_seq, d_k};
    c->k_cache = tensor_zeros(params_pool, 4, shape, 0);
    c->v_cache = tensor_zeros(params_pool, 4, shape, 0);
    c->seq_len = 0;
    c->max_seq = max_seq;
    return c;
}

/* K_new/V_new [B, H, N_new, d_k] contiguous -> rows seq_len.. of every (b, h). */
void kv_cache_append(kv_cache *c, const tensor *K_new, const tensor *V_new) {
    assert(c && K_new && V_new && K_new->ndim == 4 && V_new->ndim == 4);
    const int B = K_new->shape[0], H = K_new->shape[1], N = K_new->shape[2], D = K_new->shape[3];
    assert(B == c->k_cache->shape[0] && H == c->k_cache->shape[1] && D == c->k_cache->shape[3]);
    assert(N == V_new->shape[2]);
    assert(c->seq_len + N <= c->max_seq && "kv_cache_append: cache full");
    assert(!dnn_amd_cache_is_bound(c) && "kv_cache_append: the cache's rows live on the device (block forward)");
    const size_t row = (size_t)N * D * sizeof(float);
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++) {
            const size_t dst = (size_t)c->k_cache->offset + (size_t)b * c->k_cache->strides[0] +
                               (size_t)h * c->k_cache->strides[1] + (size_t)c->seq_len * c->k_cache->strides[2];
            const size_t src = (size_t)b * K_new->strides[0] + (size_t)h * K_new->strides[1];
            memcpy((float *)c->k_cache->data + dst, (const float *)K_new->data + K_new->offset + src, row);
            memcpy((float *)c->v_cache->data + dst, (const float *)V_new->data + V_new->offset + src, row);
        }
    c->seq_len += N;
}

tensor *kv_cache_get_K(struct mem_pool *scratch, kv_cache *c) {
    assert(c && c->seq_len > 0 && "kv_cache_get_K: empty cache");
    dnn_amd_cache_sync(c);
    return tensor_slice(scratch, c->k_cache, 2, 0, c->seq_len);
}

tensor *kv_cache_get_V(struct mem_pool *scratch, kv_cache *c) {
    assert(c && c->seq_len > 0 && "kv_cache_get_V: empty cache");
    dnn_amd_cache_sync(c);
    return tensor_slice(scratch, c->v_cache, 2, 0, c->seq_len);
}

transformer_block *transformer_block_create(struct mem_pool *params_pool, int d_model, int n_heads,
                                            int d_k, int intermediate_size) {
    assert(d_model > 0 && n_heads > 0 && d_k > 0 && intermediate_size > 0);
    assert(d_model == n_heads * d_k && "d_model must equal n_heads * d_k");
    transformer_block *b = _mem_pool_alloc(params_pool, sizeof(transformer_block), NULL);
    module_init(&b->base, params_pool, "transformer_block");
    b->d_model = d_model;
    b->n_heads = n_heads;
    b->d_k = d_k;
    b->qkv_proj = linear_create(params_pool, d_model, 3 * n_heads * d_k);
    module_add_child(&b->base, "qkv_proj", &b->qkv_proj->base);
    b->out_proj = linear_create(params_pool, n_heads * d_k, d_model);
    module_add_child(&b->base, "out_proj", &b->out_proj->base);
    b->attn_norm = rms_norm_create(params_pool, d_model, 1e-5f);
    module_add_child(&b->base, "attn_norm", &b->attn_norm->base);
    b->ffn_norm = rms_norm_create(params_pool, d_model, 1e-5f);
    module_add_child(&b->base, "ffn_norm", &b->ffn_norm->base);
    b->ffn = swiglu_ffn_create(params_pool, d_model, intermediate_size);
    module_add_child(&b->base, "ffn", &b->ffn->base);
    b->freqs_cos = b->freqs_sin = NULL;
    return b;
}

long long transformer_block_num_parameters(transformer_block *b) { return module_num_parameters(&b->base); }
