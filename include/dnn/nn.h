/* nn.h -- layer structs of the decode path (reference include/nn.h:14-98). */
#ifndef DNN_NN_H
#define DNN_NN_H
#include "tensor.h"
#include "module.h"

/* y = x @ W + b, W [in_features][out_features] */
typedef struct linear {
    module  base;
    tensor *weight;
    tensor *bias;
    int     in_features;
    int     out_features;
} linear;

typedef struct swiglu_ffn {
    module  base;
    linear *gate_proj;
    linear *up_proj;
    linear *down_proj;
    int     d_model;
    int     intermediate_size;
} swiglu_ffn;

typedef struct rms_norm {
    module  base;
    tensor *weight;
    float   eps;
    int     d;
} rms_norm;

typedef struct embedding {
    module  base;
    tensor *weight;
    int     vocab_size;
    int     d_model;
} embedding;

/* conv2d (reference nn.h:107-116): weight [out][in][k][k], bias [out].  Here
 * only as vision_lm's patch embedding (kernel = stride = patch, no padding). */
typedef struct conv2d {
    module  base;
    tensor *weight;
    tensor *bias;
    int     in_channels;
    int     out_channels;
    int     kernel_size;
    int     stride;
    int     padding;
} conv2d;

linear     *linear_create(struct mem_pool *params, int in_features, int out_features);
/* conv2d_create (nn.c:90-110): weight ~ U(-b, b), b = sqrt(6 / (in * k * k)),
 * bias 0 -- the same draws from the default stream as the reference. */
conv2d     *conv2d_create(struct mem_pool *params, int in_channels, int out_channels, int kernel_size, int stride,
                          int padding);
/* linear_forward (nn.c:27-36): x [..., in] -> x . W + b [..., out], on the
 * device (dnn_hip_linear). */
tensor     *linear_forward(struct mem_pool *scratch, linear *l, const tensor *input);
swiglu_ffn *swiglu_ffn_create(struct mem_pool *params, int d_model, int intermediate_size);
/* swiglu_ffn_forward (nn.c:61-78): x [..., d_model] -> down(SwiGLU(gate(x), up(x)))
 * [..., d_model], on the device (the three weights resident after the first
 * call). */
tensor     *swiglu_ffn_forward(struct mem_pool *scratch, swiglu_ffn *ffn, const tensor *x);
rms_norm   *rms_norm_create(struct mem_pool *params, int d, float eps);
embedding  *embedding_create(struct mem_pool *params, int vocab_size, int d_model);

/* rms_norm_forward (nn.c:169-173): y = (x * rs) * weight per row of x [..., d].
 * On the device. */
tensor *rms_norm_forward(struct mem_pool *scratch, rms_norm *norm, const tensor *x);

/* embedding_forward (nn.c:193-199 -> tensor_embedding, embedding.c:63-110):
 * ids [N] int32 -> rows [N, d_model] of the table, gathered on the device
 * (the table resident in HBM; ids outside [0, vocab) assert).  `data` is
 * unused, as in the reference. */
tensor *embedding_forward(struct mem_pool *scratch, struct mem_pool *data, embedding *emb, const tensor *ids);

long long linear_num_parameters(linear *l);
long long swiglu_ffn_num_parameters(swiglu_ffn *ffn);
long long embedding_num_parameters(embedding *emb);

#endif
