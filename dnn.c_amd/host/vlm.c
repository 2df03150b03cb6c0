/* vlm.c -- vision_lm (reference src/vlm.c): a decoder_lm fed with an image
 * prefix.  Creation and initialisation draw from the default stream in the
 * reference's order (vlm.c:20-127), so a seed gives the reference's weights.
 * The image projection runs as one device GEMM (dnn_hip_linear); the decoder
 * runs through the device layer-level path (blocks.c).  Training is not part
 * of this library. */
#include "dnn/vlm.h"
#include "dnn/rng.h"
#include "dnn/autograd.h"
#include "dnn/tokenizer.h"
#include "dnn_hip.h"
#include "device.h"
#include <assert.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

vision_lm *vision_lm_create(struct mem_pool *params_pool, int vocab_size, int d_model, int n_layers, int n_heads,
                            int d_k, int intermediate_size, int image_channels, int image_h, int image_w,
                            int patch_size, int use_image_pos) {
    assert(vocab_size > 0 && d_model > 0 && n_layers > 0);
    assert(n_heads > 0 && d_k > 0 && intermediate_size > 0);
    assert(d_model == n_heads * d_k && "d_model must equal n_heads * d_k");
    assert(image_h > 0 && image_w > 0 && patch_size > 0);
    assert(image_h % patch_size == 0 && "image_h must be divisible by patch_size");
    assert(image_w % patch_size == 0 && "image_w must be divisible by patch_size");
    vision_lm *v = _mem_pool_alloc(params_pool, sizeof(vision_lm), NULL);
    memset(v, 0, sizeof *v);
    module_init(&v->base, params_pool, "vision_lm");
    v->vocab_size = vocab_size;
    v->d_model = d_model;
    v->image_channels = image_channels;
    v->image_h = image_h;
    v->image_w = image_w;
    v->patch_size = patch_size;
    v->patch_h = image_h / patch_size;
    v->patch_w = image_w / patch_size;
    v->n_img_tokens = v->patch_h * v->patch_w;
    v->use_image_pos = use_image_pos;
    /* registration order: patch_embed, img_proj, lm, image_pos (vlm.c:49-79) */
    v->patch_embed = conv2d_create(params_pool, image_channels, d_model, patch_size, patch_size, 0);
    module_add_child(&v->base, "patch_embed", &v->patch_embed->base);
    v->img_proj = linear_create(params_pool, image_channels * patch_size * patch_size, d_model);
    module_add_child(&v->base, "img_proj", &v->img_proj->base);
    v->lm = decoder_lm_create(params_pool, vocab_size, d_model, n_layers, n_heads, d_k, intermediate_size);
    module_add_child(&v->base, "lm", &v->lm->base);
    if (use_image_pos) {
        v->image_pos = tensor_zeros(params_pool, 3, (int[]){1, v->n_img_tokens, d_model}, 1);
        module_param(&v->base, "image_pos", v->image_pos);
    }
    return v;
}

/* decoder: GPT-2 style; patch weights N(0, 1/(C*P*P)), bias 0; image_pos
 * N(0, 0.02^2); img_proj keeps its create-time draws (vlm.c:88-127). */
void vision_lm_init_weights(vision_lm *v) {
    assert(v);
    decoder_lm_init_weights(v->lm);
    const int C = v->image_channels, P = v->patch_size;
    const float std = sqrtf(1.0f / (float)(C * P * P));
    float *w = tensor_data_ptr(v->patch_embed->weight);
    for (int i = 0, n = tensor_numel(v->patch_embed->weight); i < n; i++) w[i] = dnn_rng_normal(dnn_get_rng()) * std;
    memset(tensor_data_ptr(v->patch_embed->bias), 0, sizeof(float) * (size_t)tensor_numel(v->patch_embed->bias));
    if (v->image_pos) {
        float *p = tensor_data_ptr(v->image_pos);
        for (int i = 0, n = tensor_numel(v->image_pos); i < n; i++) p[i] = dnn_rng_normal(dnn_get_rng()) * 0.02f;
    }
}

void vision_lm_enable_rope(struct mem_pool *params_pool, vision_lm *v, int max_text_len, float base) {
    assert(v);
    decoder_lm_enable_rope(params_pool, v->lm, v->n_img_tokens + max_text_len, base);
}

long long vision_lm_num_parameters(vision_lm *v) { return module_num_parameters(&v->base); }

/* [B,I,C*P*P] pre-patched rows through img_proj, or [B,C,H,W] through the
 * patch conv (kernel = stride = P, no padding: one linear map per patch, patch
 * m = py*Wp + px, patch vector c*P*P + ky*P + kx -- the conv weight's own
 * [out][C][P][P] order), vlm.c:153-186. */
tensor *vision_lm_image_embeds(struct mem_pool *scratch, vision_lm *v, const tensor *images) {
    assert(v && images);
    assert(images->contiguous && "images must be contiguous");
    const int B = images->shape[0], I = v->n_img_tokens, D = v->d_model, C = v->image_channels, P = v->patch_size;
    const int PD = C * P * P;
    if (images->ndim == 3) {
        assert(images->shape[1] == I && "patch count mismatch");
        assert(images->shape[2] == PD && "patch dim mismatch");
        return linear_forward(scratch, v->img_proj, images);
    }
    assert(images->ndim == 4 && "images must be 4D [B, C, H, W] or 3D [B, patches, patch_dim]");
    assert(images->shape[1] == C && images->shape[2] == v->image_h && images->shape[3] == v->image_w);
    const float *src = (const float *)images->data + images->offset;
    float *patches = malloc(sizeof(float) * (size_t)B * I * PD);
    assert(patches);
    const int Hh = v->image_h, Ww = v->image_w;
    for (int b = 0; b < B; b++)
        for (int py = 0; py < v->patch_h; py++)
            for (int px = 0; px < v->patch_w; px++) {
                float *row = patches + ((size_t)b * I + (size_t)py * v->patch_w + px) * PD;
                for (int c = 0; c < C; c++)
                    for (int ky = 0; ky < P; ky++)
                        memcpy(row + (size_t)c * P * P + (size_t)ky * P,
                               src + (((size_t)b * C + c) * Hh + (size_t)py * P + ky) * Ww + (size_t)px * P,
                               sizeof(float) * (size_t)P);
            }
    float *y = malloc(sizeof(float) * (size_t)B * I * D);
    assert(y);
    dnn_amd_check(dnn_hip_linear(patches, B * I, PD, tensor_data_ptr(v->patch_embed->weight), 1,
                                 tensor_data_ptr(v->patch_embed->bias), D, y),
                  "dnn_hip_linear");
    free(patches);
    /* The reference's tensor_conv2d stores its im2col GEMM result as
     * [N*Ho*Wo][out_C] under the shape [N, out_C, Ho, Wo] (conv.c:838-846),
     * and vision_lm_image_embeds then moves channels last (vlm.c:176-183).
     * Token t, dim d of image b is therefore element d*I + t of image b's
     * [I][D] block read in that order: y[b][(d*I + t) / D][(d*I + t) % D]. */
    tensor *out = tensor_scratch(scratch, 3, (int[]){B, I, D}, 0);
    float *o = tensor_data_ptr(out);
    for (int b = 0; b < B; b++)
        for (int t = 0; t < I; t++)
            for (int d = 0; d < D; d++) o[((size_t)b * I + t) * D + d] = y[(size_t)b * I * D + (size_t)d * I + t];
    free(y);
    return out;
}

tensor *vision_lm_build_embeds(struct mem_pool *scratch, vision_lm *v, const tensor *images, const tensor *text_ids) {
    assert(v && images && text_ids);
    assert(images->shape[0] == text_ids->shape[0] && "batch mismatch");
    tensor *img = vision_lm_image_embeds(scratch, v, images);
    if (v->use_image_pos && v->image_pos) {
        /* [B,I,D] + [1,I,D] (vlm.c:203-205) */
        const int B = img->shape[0], n = v->n_img_tokens * v->d_model;
        float *d = tensor_data_ptr(img);
        const float *p = tensor_data_ptr(v->image_pos);
        for (int b = 0; b < B; b++)
            for (int i = 0; i < n; i++) d[(size_t)b * n + i] = d[(size_t)b * n + i] + p[i];
    }
    tensor *txt = decoder_lm_token_embeds(scratch, v->lm, text_ids);
    return tensor_cat(scratch, img, txt, 1);
}

tensor *vision_lm_forward(struct mem_pool *scratch, vision_lm *v, const tensor *images, const tensor *text_ids) {
    tensor *e = vision_lm_build_embeds(scratch, v, images, text_ids);
    return decoder_lm_forward_embeds_ex(scratch, v->lm, e, ATTENTION_PREFIX_LM, v->n_img_tokens, NULL);
}

tensor *vision_lm_forward_text_logits(struct mem_pool *scratch, vision_lm *v, const tensor *images,
                                      const tensor *text_ids) {
    const int T = text_ids->shape[1];
    tensor *logits = vision_lm_forward(scratch, v, images, text_ids);
    return tensor_slice(scratch, logits, 1, v->n_img_tokens, T);
}

static int pick(const float *lg, int V, float temperature) {
    return temperature == 0.0f ? decoder_lm_argmax_token(lg, V) : decoder_lm_sample_with_temp(lg, V, temperature);
}

/* vlm.c:436-611: with the cache, one prefix-LM pass over image rows ++ prompt
 * (the image rows without image positions, as the reference's cached path
 * builds them), then one token per step; without it, the full forward
 * (with image positions) every step. */
int *vision_lm_generate(struct mem_pool *scratch_pool, struct mem_pool *data_pool, vision_lm *v, const tensor *image,
                        const tensor *prompt_ids, int max_new_tokens, float temperature, int use_cache, int *n_out) {
    assert(v && image && prompt_ids);
    assert((image->ndim == 4 || image->ndim == 3) && "image must be 4D [1,C,H,W] or 3D [1,patches,patch_dim]");
    assert(image->shape[0] == 1 && "only batch=1 supported");
    assert(prompt_ids->ndim == 2 && prompt_ids->shape[0] == 1 && prompt_ids->contiguous);
    assert(max_new_tokens > 0 && temperature >= 0.0f);
    const int T = prompt_ids->shape[1], max_len = T + max_new_tokens, V = v->vocab_size, D = v->d_model;
    const int I = v->n_img_tokens;
    /* the image in the data pool, so it survives scratch resets (vlm.c:484-487) */
    tensor *img_data = tensor_zeros_data(data_pool, image->ndim, image->shape);
    memcpy(tensor_data_ptr(img_data), (const float *)image->data + image->offset, sizeof(float) * (size_t)tensor_numel(image));
    image = img_data;
    int *out = _mem_pool_alloc(data_pool, sizeof(int) * (size_t)max_len, NULL);
    memcpy(out, (const int *)prompt_ids->data + prompt_ids->offset, sizeof(int) * (size_t)T);
    int cur = T;
    dnn_grad_ctx g = dnn_no_grad_enter();
    float *lg = malloc(sizeof(float) * (size_t)V);
    assert(lg);
    if (use_cache && v->lm->n_layers > 0) {
        const int H = v->lm->blocks[0]->n_heads, dk = v->lm->blocks[0]->d_k, L = v->lm->n_layers;
        const size_t mark = mem_pool_mark(data_pool);
        kv_cache **c = _mem_pool_alloc(data_pool, sizeof(kv_cache *) * (size_t)L, NULL);
        for (int l = 0; l < L; l++) c[l] = kv_cache_create(data_pool, 1, H, I + max_len, dk);
        tensor *img = vision_lm_image_embeds(scratch_pool, v, image);
        tensor *txt = decoder_lm_token_embeds(scratch_pool, v->lm, prompt_ids);
        tensor *h = tensor_cat(scratch_pool, img, txt, 1);
        for (int l = 0; l < L; l++)
            h = transformer_block_forward_cached_ex(scratch_pool, v->lm->blocks[l], h, c[l], ATTENTION_PREFIX_LM, I);
        h = rms_norm_forward(scratch_pool, v->lm->norm, h);
        tensor *logits = decoder_lm_lm_head_forward(scratch_pool, v->lm, h);
        memcpy(lg, tensor_data_ptr(logits) + (size_t)(I + T - 1) * V, sizeof(float) * (size_t)V);
        mem_pool_reset(scratch_pool);
        int id = pick(lg, V, temperature);
        out[cur++] = id;
        tensor *one = tensor_zeros_data(data_pool, 1, (int[]){1});
        while (id != TOKENIZER_EOS_ID && cur < max_len) {
            ((int *)one->data)[0] = out[cur - 1];
            tensor *e = embedding_forward(scratch_pool, NULL, v->lm->embed, one);
            tensor *x = tensor_reshape(scratch_pool, e, 3, (int[]){1, 1, D});
            for (int l = 0; l < L; l++) x = transformer_block_forward_cached(scratch_pool, v->lm->blocks[l], x, c[l]);
            x = rms_norm_forward(scratch_pool, v->lm->norm, x);
            tensor *lt = decoder_lm_lm_head_forward(scratch_pool, v->lm, x);
            memcpy(lg, tensor_data_ptr(lt), sizeof(float) * (size_t)V);
            mem_pool_reset(scratch_pool);
            id = pick(lg, V, temperature);
            out[cur++] = id;
        }
        mem_pool_release(data_pool, mark);
    } else {
        while (cur < max_len) {
            tensor *ids = tensor_zeros_data(scratch_pool, 2, (int[]){1, cur});
            memcpy(ids->data, out, sizeof(int) * (size_t)cur);
            tensor *logits = vision_lm_forward(scratch_pool, v, image, ids);
            memcpy(lg, tensor_data_ptr(logits) + (size_t)(I + cur - 1) * V, sizeof(float) * (size_t)V);
            mem_pool_reset(scratch_pool);
            const int id = pick(lg, V, temperature);
            out[cur++] = id;
            if (id == TOKENIZER_EOS_ID) break;
        }
    }
    free(lg);
    dnn_no_grad_exit(g);
    *n_out = cur;
    return out;
}
