/* vlm_main.c -- a caller of the reference's vision_lm API (vlm.h:20-171),
 * built against include/dnn and linked with libdnn_amd.so.
 *
 *   vlm_main params        the "vg" model's parameter hashes (no device use)
 *   vlm_main gen <outdir>  image embeddings of a 4D and a 3D image, the full
 *                          prefix-LM forward, and greedy vision_lm_generate
 *                          with and without the cache (device)
 *
 * The model, images and prompt are drawn exactly as tests/golden/gen_vlm.c
 * draws them from the reference, so the outputs compare with its fixtures. */
#include "dnn/dnn.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static unsigned long long fnv(const void *p, size_t n) {
    const unsigned char *b = p;
    unsigned long long h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}

static void save(const char *dir, const char *name, const float *p, size_t n) {
    char path[1024];
    snprintf(path, sizeof path, "%s/%s.f32", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, sizeof(float), n, f) != n) { perror(path); exit(1); }
    fclose(f);
}

static void ints(const char *key, const int *v, int n, int last) {
    printf("\"%s\": [", key);
    for (int i = 0; i < n; i++) printf("%s%d", i ? "," : "", v[i]);
    printf("]%s", last ? "" : ", ");
}

int main(int argc, char **argv) {
    if (argc < 2) { fprintf(stderr, "usage: vlm_main params | gen <outdir>\n"); return 2; }
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, 64 << 20, 64 << 20, 64 << 20)) return 1;
    const int V = 96, D = 128, L = 2, H = 2, F = 256, C = 3, IH = 16, IW = 16, P = 4, T = 4, NEW = 10;
    dnn_seed(6);
    vision_lm *vlm = vision_lm_create(ctx.params, V, D, L, H, D / H, F, C, IH, IW, P, 1);
    vision_lm_init_weights(vlm);
    vision_lm_enable_rope(ctx.params, vlm, 32, 10000.0f);
    int n;
    tensor **ps = module_parameters(&vlm->base, &n);
    printf("{\"params\": [");
    for (int i = 0; i < n; i++)
        printf("%s\"%016llx\"", i ? "," : "", fnv(tensor_data_ptr(ps[i]), sizeof(float) * (size_t)tensor_numel(ps[i])));
    printf("], \"n_params\": %lld", vision_lm_num_parameters(vlm));
    if (strcmp(argv[1], "gen") == 0 && argc > 2) {
        const char *dir = argv[2];
        const int I = vlm->n_img_tokens, PD = C * P * P;
        dnn_rng r = dnn_rng_seed(606);
        tensor *img4 = tensor_zeros(ctx.data, 4, (int[]){1, C, IH, IW}, 0);
        for (int i = 0; i < C * IH * IW; i++) tensor_data_ptr(img4)[i] = dnn_rng_normal(&r);
        tensor *img3 = tensor_zeros(ctx.data, 3, (int[]){1, I, PD}, 0);
        for (int i = 0; i < I * PD; i++) tensor_data_ptr(img3)[i] = dnn_rng_normal(&r);
        tensor *prompt = tensor_zeros_data(ctx.data, 2, (int[]){1, T});
        for (int i = 0; i < T; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, V);
        dnn_grad_ctx g = dnn_no_grad_enter();
        save(dir, "embeds4", tensor_data_ptr(vision_lm_image_embeds(ctx.scratch, vlm, img4)), (size_t)I * D);
        save(dir, "embeds3", tensor_data_ptr(vision_lm_image_embeds(ctx.scratch, vlm, img3)), (size_t)I * D);
        save(dir, "forward4", tensor_data_ptr(vision_lm_forward(ctx.scratch, vlm, img4, prompt)), (size_t)(I + T) * V);
        tensor *tl = vision_lm_forward_text_logits(ctx.scratch, vlm, img4, prompt);
        printf(", \"text_logits_shape\": [%d,%d,%d]", tl->shape[0], tl->shape[1], tl->shape[2]);
        mem_pool_reset(ctx.scratch);
        dnn_no_grad_exit(g);
        printf(", ");
        int no;
        int *o = vision_lm_generate(ctx.scratch, ctx.data, vlm, img4, prompt, NEW, 0.0f, 1, &no);
        ints("tokens4_cache", o, no, 0);
        o = vision_lm_generate(ctx.scratch, ctx.data, vlm, img4, prompt, NEW, 0.0f, 0, &no);
        ints("tokens4_nocache", o, no, 0);
        o = vision_lm_generate(ctx.scratch, ctx.data, vlm, img3, prompt, NEW, 0.0f, 1, &no);
        ints("tokens3_cache", o, no, 1);
    }
    printf("}\n");
    dnn_ctx_destroy(&ctx);
    return 0;
}
