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

linear     *linear_create(struct mem_pool *params, int in_features, int out_features);
swiglu_ffn *swiglu_ffn_create(struct mem_pool *params, int d_model, int intermediate_size);
rms_norm   *rms_norm_create(struct mem_pool *params, int d, float eps);
embedding  *embedding_create(struct mem_pool *params, int vocab_size, int d_model);

long long linear_num_parameters(linear *l);
long long swiglu_ffn_num_parameters(swiglu_ffn *ffn);
long long embedding_num_parameters(embedding *emb);

#endif
