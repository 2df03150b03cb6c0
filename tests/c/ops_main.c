/* ops_main.c -- a caller of the reference's op- and layer-level API that uses
 * only the reference's own declarations (ops.h, norm.h, rope.h, multihead.h,
 * nn.h, transformer.h, gpt.h), so the same file builds against the reference
 * (tests/golden/make_golden.sh: it writes the fixtures tests/golden/data/ops/)
 * and against include/dnn + libdnn_amd.so (tests/test_ops_gpu.py: every op on
 * the device).  Inputs come from the seeded default stream (tensor_randn),
 * which both libraries draw identically.
 *
 *   ops_main <outdir>     writes <outdir>/<name>.f32 for every case */
#include "dnn.h"
#include "ops.h"
#include "norm.h"
#include "rope.h"
#include "multihead.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const char *DIR_OUT;

static void save(const char *name, const tensor *t) {
    char path[1024];
    snprintf(path, sizeof path, "%s/%s.f32", DIR_OUT, name);
    FILE *f = fopen(path, "wb");
    if (!f) { perror(path); exit(1); }
    const int n = tensor_numel(t);
    const float *p = (const float *)t->data + t->offset;
    if (fwrite(p, sizeof(float), (size_t)n, f) != (size_t)n) { perror(path); exit(1); }
    fclose(f);
}

static tensor *randn(mem_pool *pool, int ndim, const int *shape) { return tensor_randn(pool, ndim, shape, 0); }

int main(int argc, char **argv) {
    if (argc < 2) return 2;
    DIR_OUT = argv[1];
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, (size_t)64 << 20, (size_t)64 << 20, (size_t)16 << 20)) return 1;
    dnn_grad_ctx g = dnn_no_grad_enter();
    dnn_seed(4242);
    mem_pool *P = ctx.params, *S = ctx.scratch;

    /* tensor_matmul_add: 2-D (both layouts), batched a with a 2-D b, broadcast batch */
    tensor *a2 = randn(S, 2, (int[]){7, 64});
    tensor *w = randn(P, 2, (int[]){64, 48});
    tensor *wt = randn(P, 2, (int[]){48, 64});
    tensor *bias = randn(P, 1, (int[]){48});
    save("mm2", tensor_matmul_add(S, a2, w, 0, bias));
    save("mm2t", tensor_matmul_add(S, a2, wt, 1, bias));
    tensor *a3 = randn(S, 3, (int[]){3, 5, 64});
    save("mm3", tensor_matmul_add(S, a3, w, 0, bias));
    tensor *b3 = randn(S, 3, (int[]){3, 64, 48});
    tensor *a1 = randn(S, 3, (int[]){1, 5, 64});
    save("mm3b", tensor_matmul_add(S, a1, b3, 0, bias));

    /* tensor_add: same shape, last-dim bias, general broadcast */
    tensor *x = randn(S, 3, (int[]){2, 3, 8});
    tensor *y = randn(S, 3, (int[]){2, 3, 8});
    tensor *bv = randn(S, 1, (int[]){8});
    tensor *bc = randn(S, 2, (int[]){3, 1});
    save("add_same", tensor_add(S, x, y));
    save("add_bias", tensor_add(S, x, bv));
    save("add_bcast", tensor_add(S, x, bc));

    /* tensor_swiglu */
    tensor *gt = randn(S, 2, (int[]){4, 100});
    tensor *up = randn(S, 2, (int[]){4, 100});
    save("swiglu", tensor_swiglu(S, gt, up));

    /* tensor_embedding */
    tensor *table = randn(P, 2, (int[]){50, 16});
    tensor *ids = tensor_zeros_data(S, 1, (int[]){7});
    const int idv[7] = {3, 0, 49, 17, 17, 8, 21};
    memcpy(ids->data, idv, sizeof idv);
    save("embedding", tensor_embedding(S, table, ids));

    /* tensor_rms_norm with and without a weight */
    tensor *xn = randn(S, 3, (int[]){3, 7, 64});
    tensor *gam = randn(P, 1, (int[]){64});
    save("rms_w", tensor_rms_norm(S, xn, gam, 1e-5f));
    save("rms_nw", tensor_rms_norm(S, xn, NULL, 1e-5f));

    /* tensor_rope on [B, H, N, d] with the reference's tables */
    tensor *fc = NULL, *fs = NULL;
    tensor_rope_freqs_init(P, &fc, &fs, 64, 16, 10000.0f);
    tensor *q = randn(S, 4, (int[]){2, 4, 9, 64});
    tensor *fc9 = tensor_slice(S, fc, 0, 0, 9), *fs9 = tensor_slice(S, fs, 0, 0, 9);
    save("rope", tensor_rope(S, q, fc9, fs9));

    /* head split / merge */
    tensor *qkv = randn(S, 3, (int[]){2, 5, 3 * 4 * 16});
    tensor *Qh, *Kh, *Vh;
    tensor_split_qkv_heads(S, qkv, 4, &Qh, &Kh, &Vh);
    save("split_q", Qh);
    save("split_k", Kh);
    save("split_v", Vh);
    save("merge", tensor_merge_heads(S, Qh));
    tensor *xh = randn(S, 3, (int[]){2, 5, 64});
    save("split_heads", tensor_split_heads(S, xh, 4));

    /* layers: linear_forward and swiglu_ffn_forward */
    linear *lin = linear_create(P, 64, 48);
    tensor *xl = randn(S, 3, (int[]){2, 3, 64});
    save("linear", linear_forward(S, lin, xl));
    swiglu_ffn *ffn = swiglu_ffn_create(P, 64, 96);
    save("ffn", swiglu_ffn_forward(S, ffn, xl));

    /* full-sequence block and hidden-state forwards of a small decoder LM
     * (d_k 64: the device kernels' head size) */
    decoder_lm *lm = decoder_lm_create(P, 64, 128, 2, 2, 64, 160);
    decoder_lm_enable_rope(P, lm, 16, 10000.0f);
    tensor *xe = randn(S, 3, (int[]){2, 9, 128});
    save("block_causal", transformer_block_forward(S, lm->blocks[0], xe));
    save("block_prefix", transformer_block_forward_ex(S, lm->blocks[1], xe, ATTENTION_PREFIX_LM, 4, NULL));
    const int lens[2] = {9, 6};
    save("block_lens", transformer_block_forward_ex(S, lm->blocks[0], xe, ATTENTION_CAUSAL, 0, lens));
    save("hidden", decoder_lm_hidden_from_embeds(S, lm, xe));
    save("hidden_prefix", decoder_lm_hidden_from_embeds_ex(S, lm, xe, ATTENTION_PREFIX_LM, 5, NULL));
    save("hidden_lens", decoder_lm_hidden_from_embeds_ex(S, lm, xe, ATTENTION_CAUSAL, 0, lens));

    dnn_no_grad_exit(g);
    printf("ok\n");
    return 0;
}
