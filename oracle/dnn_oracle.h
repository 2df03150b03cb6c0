/*
 * dnn_oracle.h -- CPU restatement of masc-it/dnn.c's GPT decode path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker.
 *
 * Every arithmetic step follows the reference's x86 NO_CBLAS scalar path in the
 * same order with the same float rounding, so that with the reference's flags
 * (gcc -O3 -ffinite-math-only -fno-signed-zeros -fno-trapping-math -fopenmp, no
 * -march) the outputs are bit-identical to the compiled reference.  That claim is
 * pinned by tests/golden (fixtures written from oracle/_ref, the reference built
 * from its own sources) -- see the per-function notes in dnn_oracle.c.
 *
 * Layouts are the reference's: linear weights are [in][out] row-major
 * (nn.h:9-20), the embedding is [V][D] and doubles as the tied lm_head
 * (gpt.c:117-122), KV caches are [H][max_seq][d_k] per layer (transformer.h:26-31).
 */
#ifndef DNN_ORACLE_H
#define DNN_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- RNG (rng.c:6-78) ---- */
typedef struct orc_rng { uint64_t s[2]; } orc_rng;
void  orc_rng_seed(orc_rng *r, uint64_t seed);
float orc_rng_uniform(orc_rng *r);
float orc_rng_normal(orc_rng *r);
int   orc_rng_uniform_int(orc_rng *r, int n);

/* ---- model ---- */
typedef struct orc_cfg {
    int V, D, L, H, dk, F;
    int max_seq;          /* RoPE table rows and KV-cache length */
    float rope_base;      /* 0 => RoPE disabled */
} orc_cfg;

typedef struct orc_layer {
    float *wqkv, *bqkv;   /* [D][3D], [3D] */
    float *wo, *bo;       /* [D][D],  [D]  */
    float *g_attn, *g_ffn;/* [D] */
    float *wg, *bg;       /* [D][F],  [F]  */
    float *wu, *bu;       /* [D][F],  [F]  */
    float *wd, *bd;       /* [F][D],  [D]  */
} orc_layer;

typedef struct orc_model {
    orc_cfg cfg;
    float *embed;         /* [V][D] */
    orc_layer *layers;    /* [L] */
    float *g_final;       /* [D] */
    float *lm_bias;       /* [V] */
    float *rope_cos, *rope_sin; /* [max_seq][dk/2] or NULL */
    float *arena;
    long long n_floats;
} orc_model;

orc_model *orc_model_create(const orc_cfg *cfg);
void orc_model_free(orc_model *m);
/* Number of parameter tensors in module-registration order and access to them. */
int    orc_model_n_params(const orc_model *m);
float *orc_model_param(orc_model *m, int i, long long *numel);

/* Seeds the default RNG and replays decoder_lm_create's draws (uniform init,
 * nn.c:10-25, nn.c:177-191, rms gamma=1 nn.c:152-167, lm_head bias 0 gpt.c:57). */
void orc_model_init_create(orc_model *m, uint64_t seed);
/* After init_create: every parameter except RMSNorm gammas <- N(0,1)*std, drawn
 * from the same default stream in module_parameters() order (module.c:123-142). */
void orc_model_init_synthetic(orc_model *m, float std);
/* decoder_lm_init_weights (gpt.c:431-477), continuing the default stream. */
void orc_model_init_gpt2(orc_model *m);
/* tensor_rope_freqs_init (rope.c:148-171). */
void orc_model_rope(orc_model *m, int max_seq, float base);

/* ---- decode state: one sequence (the reference generates batch 1 only) ---- */
typedef struct orc_state {
    const orc_model *m;
    int max_seq, seq_len;
    float *k, *v;         /* [L][H][max_seq][dk] */
    float *scratch;
} orc_state;

orc_state *orc_state_create(const orc_model *m, int max_seq);
void orc_state_free(orc_state *s);
void orc_state_reset(orc_state *s);
/* The first len cached rows of one layer's K (which 0) or V (which 1):
 * out [H][len][dk] (kv_cache_get_K/V, transformer.c:102-112). */
void orc_state_kv(const orc_state *s, int layer, int which, int len, float *out);

/* transformer_block_forward_cached_ex over all layers (transformer.c:211-416) for
 * N new rows x[N][D] (overwritten by the final hidden state, before the final
 * norm).  mode 0 = causal, 1 = prefix-LM (prefix_len rows bidirectional). */
void orc_forward_cached(orc_state *s, float *x, int N, int mode, int prefix_len);
/* final rms_norm + tied lm_head for N rows (gpt.c:357-358, 117-122). */
void orc_head(const orc_model *m, const float *x, int N, float *logits);
/* embedding gather (embedding.c:63-110). */
void orc_embed(const orc_model *m, const int *ids, int N, float *x);
/* decoder_lm_argmax_token (gpt.c:220-230). */
int  orc_argmax(const float *logits, int n);

/* decoder_lm_generate(use_cache=1, temperature=0) (gpt.c:258-375).  out gets
 * prompt + generated ids; returns n_out.  logits (nullable) receives one row of
 * V floats per generated token.  eos < 0 disables the EOS stop. */
int orc_generate(const orc_model *m, const int *prompt, int P, int max_new,
                 int eos, int *out, float *logits);

/* Full-sequence forward without cache (decoder_lm_forward, gpt.c:148-151 ->
 * transformer_block_forward_ex transformer.c:151-201 -> tensor_attention_ex
 * attention.c:671-772) for one sequence of N ids; logits [N][V]. */
void orc_forward_full(const orc_model *m, const int *ids, int N, float *logits);

/* ---- single ops, for op-level parity (same formulas as above) ---- */
void orc_matmul_add(const float *a, const float *w, const float *b, float *y,
                    int M, int K, int N, int trans_b);
void orc_rms_norm(const float *x, const float *w, float *y, int n, int d, float eps);
void orc_rope_rows(float *x, int n_rows, int d, const float *c, const float *s);
void orc_swiglu(const float *g, const float *u, float *y, int n);
/* one query row against S visible keys: o[dk] */
void orc_attend_row(const float *q, const float *k, const float *v, int S, int dk,
                    int row_stride, float *scores, float *o);

/* RoPE tables of the model ([rows][d_k/2], NULL when disabled). */
const float *orc_model_rope_cos(const orc_model *m);
const float *orc_model_rope_sin(const orc_model *m);
int orc_model_rope_rows(const orc_model *m);

/* FNV-1a 64 of a byte buffer (fixture identity of float arrays). */
uint64_t orc_fnv(const void *p, size_t n);

#ifdef __cplusplus
}
#endif
#endif
