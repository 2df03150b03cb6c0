/*
 * dnn_hip.h -- the C-ABI device layer of the MI355X (gfx950) decode path.
 *
 * Plain C: opaque handles, plain pointers and sizes, int status codes.  The host
 * library (libdnn_amd.so, the reference-compatible API declared in include/dnn/)
 * calls these; so can any FFI (ctypes, cgo, JNI) directly.
 *
 * Which reference interface each entry point serves:
 *   dnn_hip_model_create  <- the params pool as built by decoder_lm_create
 *                            (gpt.c:16-62) and filled by init/module_load; the
 *                            pointers are module_parameters() order (module.c:123-142)
 *   dnn_hip_model_rope    <- decoder_lm_enable_rope / tensor_rope_freqs_init
 *                            (gpt.c:481-496, rope.c:148-171)
 *   dnn_hip_session_*     <- kv_cache_create / the per-layer caches of
 *                            decoder_lm_generate (transformer.c:30-38, gpt.c:295-301),
 *                            extended with one sequence length per batch row
 *                            (the seq_lens convention of attention.h:39-41)
 *   dnn_hip_decode        <- the token loop of decoder_lm_generate (gpt.c:306-375):
 *                            embedding -> transformer_block_forward_cached x L
 *                            (transformer.c:211-416) -> final rms_norm -> tied
 *                            lm_head (gpt.c:117-122) -> argmax (gpt.c:220-230)
 *   dnn_hip_generate      <- decoder_lm_generate(use_cache=1, temperature=0)
 *                            (gpt.h:104-108)
 *
 * Errors: every call returns DNN_HIP_OK (0) or a negative code; the message of
 * the last failure on the calling thread is dnn_hip_last_error().  The
 * reference asserts on the same conditions (pool.c:39-40, transformer.c:55-56,
 * embedding.c:82, gpt.c:264); the host library turns a non-zero code into the
 * same fatal assert.
 *
 * Threading: a model or session is used by one host thread at a time.  All
 * calls are synchronous: results are in host memory when they return.
 */
#ifndef DNN_HIP_H
#define DNN_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DNN_HIP_OK        0
#define DNN_HIP_EINVAL   -1   /* bad argument or shape */
#define DNN_HIP_EDEVICE  -2   /* HIP runtime failure */
#define DNN_HIP_ENOMEM   -3   /* device allocation failed */
#define DNN_HIP_ERANGE   -4   /* KV cache / RoPE table / token id out of range */

typedef struct dnn_hip_model dnn_hip_model;
typedef struct dnn_hip_session dnn_hip_session;

/* Message of the last failed call on this thread ("" if none). */
const char *dnn_hip_last_error(void);

/* Selects the device for this thread; idempotent. */
int dnn_hip_init(int device);

/* Mirrors a decoder LM's parameters into HBM (one upload; call again to
 * refresh after the host weights change).  params holds 1 + 12*L + 2 pointers in
 * module_parameters() order of the reference's decoder_lm:
 *   embed.weight [V][D]
 *   per block: qkv_proj.weight [D][3D], qkv_proj.bias [3D], out_proj.weight [D][D],
 *              out_proj.bias [D], attn_norm.weight [D], ffn_norm.weight [D],
 *              ffn.gate_proj.weight [D][F], .bias [F], ffn.up_proj.weight [D][F],
 *              .bias [F], ffn.down_proj.weight [F][D], .bias [D]
 *   norm.weight [D], lm_head.bias [V]
 * eps: 2*L+1 RMSNorm epsilons (attn, ffn per block, then final) or NULL for 1e-5.
 * Requires D == H*dk and dk == 64. */
int dnn_hip_model_create(int vocab_size, int d_model, int n_layers, int n_heads,
                         int d_k, int intermediate_size,
                         const float *const *params, int n_params,
                         const float *eps, dnn_hip_model **out);

/* Weight storage of a device model. */
#define DNN_HIP_WEIGHTS_F32   0
/* Every weight matrix (embedding / tied lm_head, qkv, out, gate, up, down)
 * rounded to bf16 (round to nearest even) and streamed as bf16; biases, RMSNorm
 * gammas and all arithmetic stay fp32 (W16A32).  The reference is fp32-only:
 * this is the fp32 model on bf16-rounded weights.  Decode of such a model runs
 * on the batched engine. */
#define DNN_HIP_WEIGHTS_BF16  1

/* dnn_hip_model_create with a choice of weight storage (DNN_HIP_WEIGHTS_*). */
int dnn_hip_model_create_ex(int vocab_size, int d_model, int n_layers, int n_heads,
                            int d_k, int intermediate_size,
                            const float *const *params, int n_params,
                            const float *eps, int weights, dnn_hip_model **out);

/* Re-uploads the parameters of an existing model (same shapes). */
int dnn_hip_model_update(dnn_hip_model *m, const float *const *params, int n_params);

/* Installs the RoPE tables cos/sin [rows][d_k/2] (NULL disables RoPE). */
int dnn_hip_model_rope(dnn_hip_model *m, const float *cos_table,
                       const float *sin_table, int rows);

int dnn_hip_model_destroy(dnn_hip_model *m);

/* A decode session: the per-layer KV caches of `batch` rows in HBM (K stored
 * transposed, [L][B][H][d_k][max_seq]; V as [L][B][H][max_seq][d_k]) plus the
 * exchange arena of the decode kernel.  Every row starts empty.
 * 1 <= batch <= 64.  Sessions of at most 4 fp32 rows decode with one
 * persistent kernel launch per call; sessions of more rows (and every session
 * of a bf16 model) decode on the batched engine, one replay of a captured HIP
 * graph per step, every weight read once per step for all rows (the
 * persistent kernel takes up to 8 rows when DNN_HIP_DECODE_KERNEL=3). */
int dnn_hip_session_create(dnn_hip_model *m, int batch, int max_seq,
                           dnn_hip_session **out);
/* Empties every row (lengths back to 0). */
int dnn_hip_session_reset(dnn_hip_session *s);
/* Current cached length of each row -> lens[batch]. */
int dnn_hip_session_lengths(dnn_hip_session *s, int *lens);
int dnn_hip_session_destroy(dnn_hip_session *s);

/* Runs n_steps decode steps on every row.  Step t of row b feeds
 *   feed[t*batch + b]          while t < n_feed[b]   (n_feed NULL: n_feed_all)
 *   the argmax of step t-1     afterwards (greedy)
 * and appends one position to the row.  ids[t*batch + b] (nullable) receives the
 * argmax of step t (first index of the maximum, as gpt.c:220-230); logits
 * (nullable) receives the [n_steps][batch][V] rows.  With eos >= 0 the loop
 * ends early once every row has produced eos in its greedy part; *steps_done
 * (nullable) gets the number of steps run.  Requires n_feed >= 1 per row and
 * length + n_steps <= max_seq (and <= RoPE rows). */
int dnn_hip_decode(dnn_hip_session *s, const int *feed, int n_feed_all,
                   const int *n_feed, int n_steps, int eos, int *ids,
                   float *logits, int *steps_done);

/* Multi-token cached prefill of every row: transformer_block_forward_cached_ex
 * over all layers for N new rows per sequence (transformer.c:211-416, the
 * multi-token form of the prompt loop gpt.c:306-344, and the prefix prefill of
 * vision_lm_generate vlm.c:497-517), then the final rms_norm, tied lm_head and
 * argmax of each row's last new position.
 *   row b's new rows: n_embed input rows embeds[b][0..n_embed)[d_model] (e.g.
 *   image patch embeddings; NULL when n_embed = 0), then n_ids[b] tokens
 *   ids[b * n_ids_max + t] (n_ids NULL: n_ids_max each), embedded by the model.
 *   mode 0: causal (row at position p sees keys <= p); mode 1: prefix-LM
 *   (ATTENTION_PREFIX_LM, transformer.c:313-323: a row at p < prefix_len sees
 *   keys < prefix_len, later rows keys <= p), which needs empty rows.
 * next_ids[b] gets the argmax of row b's last new position, logits (nullable)
 * [batch][V] its logits.  Each row's length grows by its new rows; a following
 * dnn_hip_decode(s, next_ids, 1, ...) continues greedily. */
int dnn_hip_prefill(dnn_hip_session *s, const float *embeds, int n_embed,
                    const int *ids, int n_ids_max, const int *n_ids,
                    int mode, int prefix_len, int *next_ids, float *logits);

/* One transformer block -- layer `layer` of the model -- over n_new new rows of
 * every batch row at positions [pos0, pos0 + n_new): transformer_block_forward_cached_ex
 * (transformer.c:211-416) with the reference's per-layer kv_cache whose
 * seq_len is pos0.  Appends the rows' K/V to the session's layer cache, attends
 * over positions [0, pos0 + n_new) (mode / prefix_len as dnn_hip_prefill; mode 1
 * needs pos0 = 0).  x and y: host [batch][n_new][d_model].  The session's
 * lengths are not changed: the caller's cache lengths are the positions. */
int dnn_hip_block_forward(dnn_hip_session *s, int layer, const float *x, int n_new,
                          int pos0, int mode, int prefix_len, float *y);

/* The tied lm_head over n rows x [n][d_model]: logits [n][V] = (norm ?
 * rms_norm(x) with the final gamma : x) . embed^T + lm_head bias.  norm = 0 is
 * decoder_lm_lm_head_forward (gpt.c:117-122); norm = 1 adds the final
 * rms_norm_forward before it (gpt.c:357-358). */
int dnn_hip_head_forward(dnn_hip_session *s, const float *x, int n, int norm, float *logits);

/* Embedding rows of n token ids: out [n][d_model] (embedding.c:63-110; ids
 * outside [0, V) are DNN_HIP_ERANGE, where the reference asserts). */
int dnn_hip_embed(dnn_hip_session *s, const int *ids, int n, float *out);

/* rms_norm of n rows x [n][d] with gamma [d]: y = (x * rs) * gamma, rs =
 * 1/sqrtf(sum(x^2)/d + eps) (tensor_rms_norm, norm.c:404-495).  d <= d_model. */
int dnn_hip_rms_norm(dnn_hip_session *s, const float *x, const float *gamma, int n, int d,
                     float eps, float *y);

/* The first len cached positions of one layer's K (which = 0) or V (which = 1)
 * in the reference's kv_cache layout: out [batch][H][len][d_k]
 * (kv_cache_get_K / kv_cache_get_V, transformer.c:90-112). */
int dnn_hip_cache_read(dnn_hip_session *s, int layer, int which, int len, float *out);

/* y [n][out] = x [n][in] . W + b on the device -- linear_forward (nn.c:27-36,
 * tensor_matmul_add) for weights the caller holds: w_layout 0 = W [in][out]
 * (the reference's linear), 1 = W [out][in] (a conv2d weight [out][C][k][k]
 * flattened, as vision_lm's patch embedding uses it, vlm.c:175-186).  b may be
 * NULL.  x, W, b, y are host memory; synchronous.  W stays resident on the
 * device (dnn_hip_op_linear with cache_w = 1). */
int dnn_hip_linear(const float *x, int n, int in, const float *w, int w_layout, const float *b, int out,
                   float *y);

/* ---- op level ------------------------------------------------------------
 * The reference's tensor ops (ops.h, norm.h, rope.h, multihead.h) and its
 * linear / SwiGLU FFN layers, on host tensors, computed on the device.  No
 * model or session is needed; every call is synchronous (the result is in
 * host memory when it returns) and serialised per device.  Operands marked
 * cacheable (cache_* = 1: layer weights, embedding tables -- tensors that live
 * as long as a params pool) stay resident in HBM after their first upload,
 * keyed by host pointer, element count and a fingerprint of 4,096 sampled
 * values; an in-place edit missing every sample needs dnn_hip_op_cache_drop.
 * The matmul, the elementwise add, RoPE, the gather and the layout ops sum and
 * round as the reference's NO_CBLAS loops do (k in order, bias last, no FMA
 * contraction), so their results are the reference's bits. */

#define DNN_HIP_VIEW_MAX_DIMS 8
/* A strided view of host floats: element (i0, ..., i_{ndim-1}) is
 * data[sum_d i_d * strides[d]] (the reference tensor's shape / strides, data
 * already advanced by its offset).  Strides are non-negative. */
typedef struct dnn_hip_view {
    const float *data;
    int ndim;
    int shape[DNN_HIP_VIEW_MAX_DIMS];
    int strides[DNN_HIP_VIEW_MAX_DIMS];
} dnn_hip_view;

/* tensor_matmul_add (ops.h:21, ops_matrix.c:964-1183): out = a . b + bias, or
 * a . b^T + bias with trans_b; a [..., M, K], b [..., K, N] ([..., N, K] with
 * trans_b), leading (batch) dimensions broadcast; bias [N] (required, as in
 * the reference).  out: contiguous [batch..., M, N]. */
int dnn_hip_op_matmul_add(const dnn_hip_view *a, const dnn_hip_view *b, int trans_b, const float *bias,
                          int cache_b, float *out);
/* tensor_add (ops.h:7, ops_elem.c:110-175): out = a + b with right-aligned
 * broadcasting; out: contiguous, the broadcast shape. */
int dnn_hip_op_add(const dnn_hip_view *a, const dnn_hip_view *b, float *out);
/* tensor_swiglu (ops.h:29, ops_activation.c:283-333): out = (g / (1 + e^-g)) * u,
 * broadcast as tensor_add. */
int dnn_hip_op_swiglu(const dnn_hip_view *gate, const dnn_hip_view *up, float *out);
/* tensor_rms_norm (norm.h:35, norm.c:404-495): y = (x * rs) * gamma per row of
 * n rows x d, rs = 1/sqrtf(sum(x^2) * (1/d) + eps); gamma NULL means 1. */
int dnn_hip_op_rms_norm(const float *x, int n, int d, const float *gamma, float eps, float *y);
/* tensor_rope (rope.h:27, rope.c:92-144): x [outer][N][d] rotated in place,
 * pair k of row n by cos_t/sin_t [N][d/2]. */
int dnn_hip_op_rope(float *x, int outer, int N, int d, const float *cos_t, const float *sin_t);
/* tensor_embedding (ops.h:63, embedding.c:63-110): out [n][D] = table[ids[i]]
 * (table [V][D]; an id outside [0, V) is DNN_HIP_ERANGE, where the reference
 * asserts). */
int dnn_hip_op_embedding(const float *table, int V, int D, int cache_table, const int *ids, int n, float *out);
/* tensor_split_qkv_heads (multihead.h:33): x [B][N][3*H*dk] -> out0/1/2
 * [B][H][N][dk] (parts = 3); tensor_split_heads (multihead.h:20): x
 * [B][N][H*dk] -> out0 [B][H][N][dk] (parts = 1). */
int dnn_hip_op_split_heads(const float *x, int B, int N, int H, int dk, int parts, float *out0, float *out1,
                           float *out2);
/* tensor_merge_heads (multihead.h:21): x [B][H][N][dk] -> out [B][N][H*dk]. */
int dnn_hip_op_merge_heads(const float *x, int B, int H, int N, int dk, float *out);
/* linear_forward (nn.h:23, nn.c:27-36): y [n][out] = x [n][in] . W + b, W
 * [in][out] (w_layout 0) or [out][in] (1); b may be NULL (zero). */
int dnn_hip_op_linear(const float *x, int n, int in, const float *w, int w_layout, const float *b, int out,
                      int cache_w, float *y);
/* swiglu_ffn_forward (nn.h:45, nn.c:61-78): y [n][d_model] = down(SwiGLU(gate(x),
 * up(x))), weights [in][out] as the reference's linears (resident after the
 * first call), biases required. */
int dnn_hip_op_swiglu_ffn(const float *x, int n, int d_model, int d_ffn, const float *wg, const float *bg,
                          const float *wu, const float *bu, const float *wd, const float *bd, float *y);
/* Drops the resident copy of one cached host operand (NULL: all of them). */
int dnn_hip_op_cache_drop(const float *host);

/* decoder_lm_generate(use_cache=1, temperature=0) for one sequence: out gets
 * prompt + generated ids (P + max_new ints), *n_out its length (stops after eos
 * when eos >= 0).  Uses a fresh session of max_seq = P + max_new. */
int dnn_hip_generate(dnn_hip_model *m, const int *prompt, int n_prompt,
                     int max_new, int eos, int *out, int *n_out);

/* Device time of the last dnn_hip_decode call on this session, in ms, measured
 * with HIP events around its kernel launches on the session's stream. */
int dnn_hip_session_last_ms(dnn_hip_session *s, float *ms);

/* Number of workgroups the persistent decode kernel runs with on this session
 * (0 = one per compute unit, the default; larger values are capped there) --
 * a tuning knob. */
int dnn_hip_session_set_grid(dnn_hip_session *s, int n_workgroups);
/* Workgroups the last dnn_hip_decode launch on this session used. */
int dnn_hip_session_grid(dnn_hip_session *s, int *n_workgroups);
/* Which decode path the last dnn_hip_decode call used: 3 = the persistent
 * kernel (up to 4 rows by default, up to 8 when DNN_HIP_DECODE_KERNEL=3 at
 * session creation), 6 = the batched engine (more rows, bf16 weights, or
 * DNN_HIP_DECODE_KERNEL=6). */
int dnn_hip_session_kernel(dnn_hip_session *s, int *which);
/* Workgroups per (row, head) over which the last decode call split each
 * head's cached keys, on the persistent kernel (3) or the batched engine (6); 1 on
 * the other paths (1 = unsplit; chosen from the call's longest history, or
 * fixed by the environment variable DNN_HIP_ATT_SPLITS at session creation). */
int dnn_hip_session_att_splits(dnn_hip_session *s, int *splits);

/* ---- decode without allocation (no counterpart in the reference) ----------
 * For callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc: the
 * persistent decode kernel of dnn_hip_decode on buffers the caller owns, its
 * scratch (exchange arena and status words) in a fixed device array of the
 * library (DNN_HIP_STATIC_EXCHANGE_PAIRS pairs of 8 bytes, held on each GPU
 * the library runs on until the process ends).  Nothing is allocated and the
 * host is not synchronised: the work is enqueued on `stream` (a hipStream_t;
 * NULL = the null stream).  Every call on one GPU shares that array, so calls
 * that overlap on one GPU race; run them on one stream (or order them). */
#define DNN_HIP_STATIC_EXCHANGE_PAIRS ((size_t)1 << 20)

/* Floats in each of the K and V cache buffers a dnn_hip_decode_static call
 * of this model, batch and max_seq reads and writes (0 on bad arguments). */
size_t dnn_hip_kv_floats(const dnn_hip_model *m, int batch, int max_seq);

/* dnn_hip_decode's greedy loop for 1..8 rows of an fp32-weight model, every
 * buffer on the device and owned by the caller:
 *   kc, vc     K and V caches of dnn_hip_kv_floats(m, batch, max_seq) floats
 *              each (no initialisation needed)
 *   pos        [batch] cached length of each row, advanced by the steps run
 *   feed       [n_feed_rows][batch], n_feed [batch]: as dnn_hip_decode
 *   ids        [n_steps][batch] greedy ids; logits [n_steps][batch][V] or NULL
 *   max_len    a bound the caller guarantees: every row's length + n_steps <=
 *              max_len <= max_seq (and <= the RoPE rows); it sizes the
 *              attention split, and a row past it stops the launch with error
 *              bit 2 before anything is written
 * Sizes beyond the static arena (model and batch needing more than
 * DNN_HIP_STATIC_EXCHANGE_PAIRS pairs) are DNN_HIP_EINVAL.  The device status
 * of the last call is read with dnn_hip_decode_static_status. */
int dnn_hip_decode_static(dnn_hip_model *m, int batch, int max_seq, float *kc, float *vc, int *pos,
                          const int *feed, const int *n_feed, int n_steps, int eos, int max_len, int *ids,
                          float *logits, void *stream);
/* Waits for `stream`, then reports the last dnn_hip_decode_static call on the
 * current device: *steps_done (steps run; fewer when every row hit eos) and
 * *err_bits (1: a dependency wait timed out, 2: a row had no room); returns
 * DNN_HIP_EDEVICE when an error bit is set. */
int dnn_hip_decode_static_status(void *stream, int *steps_done, int *err_bits);

#ifdef __cplusplus
}
#endif
#endif
