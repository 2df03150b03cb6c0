/* transformer.h -- KV cache and pre-norm block (reference include/transformer.h:26-131). */
#ifndef DNN_TRANSFORMER_H
#define DNN_TRANSFORMER_H
#include "tensor.h"
#include "module.h"
#include "nn.h"
#include "attention.h"

typedef struct {
    tensor *k_cache;   /* [B, H, max_seq, d_k] */
    tensor *v_cache;   /* [B, H, max_seq, d_k] */
    int     seq_len;
    int     max_seq;
} kv_cache;

kv_cache *kv_cache_create(struct mem_pool *params_pool, int B, int H, int max_seq, int d_k);
void      kv_cache_append(kv_cache *kvc, const tensor *K_new, const tensor *V_new);
tensor   *kv_cache_get_K(struct mem_pool *scratch, kv_cache *kvc);
tensor   *kv_cache_get_V(struct mem_pool *scratch, kv_cache *kvc);

typedef struct {
    module      base;
    linear     *qkv_proj;
    linear     *out_proj;
    int         n_heads;
    int         d_k;
    int         d_model;
    rms_norm   *attn_norm;
    rms_norm   *ffn_norm;
    swiglu_ffn *ffn;
    tensor     *freqs_cos;   /* [max_seq_len, d_k/2] or NULL */
    tensor     *freqs_sin;
} transformer_block;

transformer_block *transformer_block_create(struct mem_pool *params_pool, int d_model, int n_heads,
                                            int d_k, int intermediate_size);
long long transformer_block_num_parameters(transformer_block *block);
/* Full-sequence forward of one block (transformer.c:151-208) over x [B, N,
 * d_model] (contiguous): attention over the N rows themselves with the mode's
 * mask (ATTENTION_CAUSAL, or ATTENTION_PREFIX_LM with prefix_len
 * bidirectional rows), no cache.  seq_lens (nullable, [B]): row b is a
 * sequence of its first seq_lens[b] rows; the rows after it, which the
 * reference leaves uncomputed (attention.c:272-285), come back zero.  Runs on
 * the device; the block must belong to a decoder_lm built by
 * decoder_lm_create. */
tensor *transformer_block_forward_ex(struct mem_pool *scratch, transformer_block *block, const tensor *x,
                                     attention_mode mode, int prefix_len, const int *seq_lens);
/* Causal full-sequence forward (transformer.c:204-208). */
tensor *transformer_block_forward(struct mem_pool *scratch, transformer_block *block, const tensor *x);

/* Cached forward of one block over x [B, N_new, d_model] (contiguous): appends
 * the new K/V to cache and attends over its rows (transformer.c:211-426).
 * Runs on the device; the block must belong to a decoder_lm built by
 * decoder_lm_create.  mode ATTENTION_PREFIX_LM needs an empty cache. */
tensor *transformer_block_forward_cached_ex(struct mem_pool *scratch, transformer_block *block,
                                            const tensor *x, kv_cache *cache,
                                            attention_mode mode, int prefix_len);
tensor *transformer_block_forward_cached(struct mem_pool *scratch, transformer_block *block,
                                         const tensor *x, kv_cache *cache);

#endif
