/*
 * gen_vlm.c -- writes tests/golden/data/vlm_gen.json (+ .f32 files) by running
 * the REAL reference's vision_lm API (vlm.c, compiled from /root/reference/src
 * into oracle/_ref/libdnnref.so by oracle/Makefile).  Dev container only; the
 * fixtures are committed data.  Build + run: tests/golden/make_golden.sh
 *
 * Model "vg": vocab 96, d_model 128, 2 layers, 2 heads, d_ffn 256, 3x16x16
 * images in 4x4 patches (16 image tokens), learned image positions; seed 6,
 * vision_lm_init_weights, RoPE for 32 text positions.
 */
#include "dnn.h"
#include "gpt.h"
#include "vlm.h"
#include "autograd.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const char *OUT = "tests/golden/data";
static FILE *J;
static int first_key = 1;

static uint64_t fnv(const void *p, size_t n) {
    const unsigned char *b = p;
    uint64_t h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}
static void key(const char *k) { fprintf(J, "%s\n\"%s\": ", first_key ? "" : ",", k); first_key = 0; }
static void j_ints(const char *k, const int *v, int n) {
    key(k); fputc('[', J);
    for (int i = 0; i < n; i++) fprintf(J, "%s%d", i ? "," : "", v[i]);
    fputc(']', J);
}
static void j_floats(const char *k, const float *v, int n) {   /* exact: bit patterns */
    key(k); fputc('[', J);
    for (int i = 0; i < n; i++) { uint32_t u; memcpy(&u, &v[i], 4); fprintf(J, "%s%u", i ? "," : "", u); }
    fputc(']', J);
}
static void bin(const char *name, const void *p, size_t n) {
    char path[512]; snprintf(path, sizeof path, "%s/%s", OUT, name);
    FILE *f = fopen(path, "wb"); fwrite(p, 1, n, f); fclose(f);
}

int main(void) {
    char path[512]; snprintf(path, sizeof path, "%s/vlm_gen.json", OUT);
    J = fopen(path, "w");
    if (!J) { perror(path); return 1; }
    fputc('{', J);
    dnn_ctx ctx;
    if (dnn_ctx_init(&ctx, (size_t)64 << 20, (size_t)64 << 20, (size_t)64 << 20)) return 1;

    const int V = 96, D = 128, L = 2, H = 2, F = 256, C = 3, IH = 16, IW = 16, P = 4, T = 4, NEW = 10;
    dnn_seed(6);
    vision_lm *vlm = vision_lm_create(ctx.params, V, D, L, H, D / H, F, C, IH, IW, P, 1);
    vision_lm_init_weights(vlm);
    vision_lm_enable_rope(ctx.params, vlm, 32, 10000.0f);
    int n;
    tensor **ps = module_parameters(&vlm->base, &n);
    key("vg_params"); fputc('[', J);
    for (int i = 0; i < n; i++)
        fprintf(J, "%s\"%016llx\"", i ? "," : "",
                (unsigned long long)fnv(tensor_data_ptr(ps[i]), (size_t)tensor_numel(ps[i]) * 4));
    fputc(']', J);
    const int I = vlm->n_img_tokens, PD = C * P * P;

    /* a 4D image and a pre-patched 3D one, N(0,1); a 4-id prompt */
    dnn_rng r = dnn_rng_seed(606);
    tensor *img4 = tensor_zeros(ctx.data, 4, (int[]){1, C, IH, IW}, 0);
    for (int i = 0; i < C * IH * IW; i++) tensor_data_ptr(img4)[i] = dnn_rng_normal(&r);
    tensor *img3 = tensor_zeros(ctx.data, 3, (int[]){1, I, PD}, 0);
    for (int i = 0; i < I * PD; i++) tensor_data_ptr(img3)[i] = dnn_rng_normal(&r);
    tensor *prompt = tensor_zeros_data(ctx.data, 2, (int[]){1, T});
    for (int i = 0; i < T; i++) ((int *)prompt->data)[i] = dnn_rng_uniform_int(&r, V);
    j_floats("vg_img4", tensor_data_ptr(img4), C * IH * IW);
    j_floats("vg_img3", tensor_data_ptr(img3), I * PD);
    j_ints("vg_prompt", (int *)prompt->data, T);

    dnn_grad_ctx g = dnn_no_grad_enter();
    tensor *e4 = vision_lm_image_embeds(ctx.scratch, vlm, img4);
    bin("vg_embeds4.f32", tensor_data_ptr(e4), sizeof(float) * I * D);
    tensor *e3 = vision_lm_image_embeds(ctx.scratch, vlm, img3);
    bin("vg_embeds3.f32", tensor_data_ptr(e3), sizeof(float) * I * D);
    tensor *lg = vision_lm_forward(ctx.scratch, vlm, img4, prompt);
    bin("vg_forward4.f32", tensor_data_ptr(lg), sizeof(float) * (I + T) * V);
    mem_pool_reset(ctx.scratch);
    dnn_no_grad_exit(g);

    int no;
    int *o = vision_lm_generate(ctx.scratch, ctx.data, vlm, img4, prompt, NEW, 0.0f, 1, &no);
    j_ints("vg_tokens4_cache", o, no);
    o = vision_lm_generate(ctx.scratch, ctx.data, vlm, img4, prompt, NEW, 0.0f, 0, &no);
    j_ints("vg_tokens4_nocache", o, no);
    o = vision_lm_generate(ctx.scratch, ctx.data, vlm, img3, prompt, NEW, 0.0f, 1, &no);
    j_ints("vg_tokens3_cache", o, no);

    fputs("\n}\n", J);
    fclose(J);
    dnn_ctx_destroy(&ctx);
    return 0;
}
