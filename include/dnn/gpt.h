/* gpt.h -- decoder-only LM (reference include/gpt.h:20-118): construction,
 * initialisation, RoPE, and the generation loop, which runs on the MI355X
 * through include/dnn_hip.h.  The training step of the reference is not part
 * of this library. */
#ifndef DNN_GPT_H
#define DNN_GPT_H
#include "tensor.h"
#include "module.h"
#include "nn.h"
#include "transformer.h"

typedef struct {
    module               base;
    embedding           *embed;
    transformer_block  **blocks;
    int                  n_layers;
    rms_norm            *norm;
    linear              *lm_head;     /* weight NULL: tied to embed->weight */
    int                  d_model;
    int                  vocab_size;
} decoder_lm;

decoder_lm *decoder_lm_create(struct mem_pool *params_pool, int vocab_size, int d_model,
                              int n_layers, int n_heads, int d_k, int intermediate_size);
void        decoder_lm_init_weights(decoder_lm *lm);
void        decoder_lm_enable_rope(struct mem_pool *params_pool, decoder_lm *lm, int max_seq_len, float base);
long long   decoder_lm_num_parameters(decoder_lm *lm);

int decoder_lm_argmax_token(const float *logits, int vocab_size);

/* h [..., d_model] -> logits [..., V] = h . embed^T + lm_head bias (the tied
 * head, gpt.c:117-122; no final norm).  On the device. */
tensor *decoder_lm_lm_head_forward(struct mem_pool *scratch, decoder_lm *lm, const tensor *h);
/* input_ids [B, N] int32 -> embeddings [B, N, d_model] (gpt.c:66-81). */
tensor *decoder_lm_token_embeds(struct mem_pool *scratch, decoder_lm *lm, const tensor *input_ids);
/* embeds [B, S, d_model] -> logits [B, S, V]: every block (full-sequence
 * attention with the mode's mask), final rms_norm, tied lm_head
 * (gpt.c:84-144).  seq_lens (or NULL) gives each batch row's valid length: its
 * rows at or past that length are not computed by the reference
 * (attention.c:272-285); here they come back as zero logits.  On the device. */
tensor *decoder_lm_forward_embeds_ex(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds,
                                     attention_mode mode, int prefix_len, const int *seq_lens);
tensor *decoder_lm_forward_embeds(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds);
/* embeds [B, S, d_model] -> the final normalised hidden state [B, S, d_model]
 * (every block, then the final rms_norm; gpt.c:84-113), seq_lens as in
 * decoder_lm_forward_embeds_ex (rows past a row's length come back zero).  On
 * the device. */
tensor *decoder_lm_hidden_from_embeds_ex(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds,
                                         attention_mode mode, int prefix_len, const int *seq_lens);
tensor *decoder_lm_hidden_from_embeds(struct mem_pool *scratch, decoder_lm *lm, const tensor *embeds);
/* input_ids [B, N] int32 -> logits [B, N, V]: full causal forward (gpt.c:148-151).
 * On the device. */
tensor *decoder_lm_forward(struct mem_pool *scratch, decoder_lm *lm, const tensor *input_ids);
int decoder_lm_sample_with_temp(const float *logits, int vocab_size, float temp);

/* Greedy (temperature 0) or sampled generation.  prompt_ids [1, N] int32.
 * Returns prompt + generated ids from data_pool; *n_out = their count. */
int *decoder_lm_generate(struct mem_pool *scratch_pool, struct mem_pool *data_pool,
                         decoder_lm *lm, const tensor *prompt_ids,
                         int max_new_tokens, float temperature, int use_cache, int *n_out);

/* ---- device mirror control (no counterpart in the reference) ----
 * The first generate call mirrors the parameters into HBM; later calls
 * re-upload when the sampled fingerprint of the host weights changed.
 * decoder_lm_device_sync forces a re-upload (e.g. after editing a few
 * weights in place); decoder_lm_device_release frees the mirror. */
void decoder_lm_device_sync(decoder_lm *lm);
void decoder_lm_device_release(decoder_lm *lm);
/* The mirror itself, for callers that drive sessions through include/dnn_hip.h
 * (batched decode, timing).  Owned by the library. */
struct dnn_hip_model *decoder_lm_device_model(decoder_lm *lm);
/* A mirror with a choice of weight storage: 0 = fp32 (the one generate uses),
 * 1 = bf16-rounded weight matrices (DNN_HIP_WEIGHTS_BF16 of dnn_hip.h). */
struct dnn_hip_model *decoder_lm_device_model_ex(decoder_lm *lm, int weights);

/* Synthetic initialisation used by the parity and bench configurations (no
 * counterpart in the reference): every parameter except the RMSNorm gammas is
 * redrawn as dnn_rng_normal() * std from the default stream, in
 * module_parameters() order. */
void decoder_lm_init_normal(decoder_lm *lm, float std);

#endif
