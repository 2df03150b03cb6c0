/* vlm.h -- the reference's prefix-LM vision-language model (include/vlm.h:20-171):
 * same struct layout and functions, minus training.  The decoder runs on the
 * MI355X through the layer-level device path; the image projection (conv2d
 * patchify or img_proj linear) is one device GEMM per image. */
#ifndef DNN_VLM_H
#define DNN_VLM_H
#include "tensor.h"
#include "module.h"
#include "nn.h"
#include "gpt.h"
#include "attention.h"

typedef struct vision_lm {
    module      base;
    decoder_lm *lm;               /* text decoder: token embed, blocks, norm, tied lm_head */
    conv2d     *patch_embed;      /* 4D image input [B,C,H,W] */
    linear     *img_proj;         /* 3D pre-patched input [B,I,C*P*P] */
    tensor     *image_pos;        /* [1, n_img_tokens, d_model] or NULL */
    int use_image_pos;
    int image_channels;
    int image_h;
    int image_w;
    int patch_size;
    int patch_h;
    int patch_w;
    int n_img_tokens;
    int d_model;
    int vocab_size;
} vision_lm;

vision_lm *vision_lm_create(struct mem_pool *params_pool, int vocab_size, int d_model, int n_layers, int n_heads,
                            int d_k, int intermediate_size, int image_channels, int image_h, int image_w,
                            int patch_size, int use_image_pos);
void       vision_lm_init_weights(vision_lm *vlm);
void       vision_lm_enable_rope(struct mem_pool *params_pool, vision_lm *vlm, int max_text_len, float base);
long long  vision_lm_num_parameters(vision_lm *vlm);
/* images [B,C,H,W] or [B,I,C*P*P] -> [B,I,d_model] (no image positions). */
tensor    *vision_lm_image_embeds(struct mem_pool *scratch, vision_lm *vlm, const tensor *images);
/* [image rows (+ image positions)] ++ [token rows] -> [B, I+T, d_model]. */
tensor    *vision_lm_build_embeds(struct mem_pool *scratch, vision_lm *vlm, const tensor *images,
                                  const tensor *text_ids);
/* logits [B, I+T, V], prefix-LM attention over the I image rows. */
tensor    *vision_lm_forward(struct mem_pool *scratch, vision_lm *vlm, const tensor *images, const tensor *text_ids);
/* logits [B, T, V] of the text positions. */
tensor    *vision_lm_forward_text_logits(struct mem_pool *scratch, vision_lm *vlm, const tensor *images,
                                         const tensor *text_ids);
/* image [1,C,H,W] or [1,I,C*P*P], prompt_ids [1,T]: prompt + generated ids from
 * data_pool (the image prefix is implicit), *n_out their count. */
int       *vision_lm_generate(struct mem_pool *scratch_pool, struct mem_pool *data_pool, vision_lm *vlm,
                              const tensor *image, const tensor *prompt_ids, int max_new_tokens, float temperature,
                              int use_cache, int *n_out);

#endif
