/* nn.c -- layer construction for the decode path (reference src/nn.c:10-25,
 * 40-59, 152-167, 177-191).  Creation order and bounds are the reference's, so
 * the same dnn_seed() yields the same weights. */
#include "dnn/nn.h"
#include "dnn/ops.h"
#include "dnn/norm.h"
#include "dnn_hip.h"
#include "device.h"
#include <assert.h>
#include <math.h>
#include <string.h>

linear *linear_create(struct mem_pool *params, int in_features, int out_features) {
    assert(in_features > 0 && out_features > 0);
    linear *l = _mem_pool_alloc(params, sizeof(linear), NULL);
    module_init(&l->base, params, "linear");
    l->in_features = in_features;
    l->out_features = out_features;
    const float bound = 1.0f / sqrtf((float)in_features);
    l->weight = tensor_uniform(params, 2, (int[]){in_features, out_features}, 1, bound);
    l->bias = tensor_uniform(params, 1, (int[]){out_features}, 1, bound);
    module_param(&l->base, "weight", l->weight);
    module_param(&l->base, "bias", l->bias);
    return l;
}

conv2d *conv2d_create(struct mem_pool *params, int in_channels, int out_channels, int kernel_size, int stride,
                      int padding) {
    assert(in_channels > 0 && out_channels > 0 && kernel_size > 0);
    conv2d *c = _mem_pool_alloc(params, sizeof(conv2d), NULL);
    module_init(&c->base, params, "conv2d");
    c->in_channels = in_channels;
    c->out_channels = out_channels;
    c->kernel_size = kernel_size;
    c->stride = stride;
    c->padding = padding;
    const float bound = sqrtf(6.0f / (float)(in_channels * kernel_size * kernel_size));
    c->weight = tensor_uniform(params, 4, (int[]){out_channels, in_channels, kernel_size, kernel_size}, 1, bound);
    c->bias = tensor_zeros(params, 1, (int[]){out_channels}, 1);
    module_param(&c->base, "weight", c->weight);
    module_param(&c->base, "bias", c->bias);
    return c;
}

tensor *linear_forward(struct mem_pool *scratch, linear *l, const tensor *input) {
    assert(l && input);
    assert(input->ndim >= 2 && "linear_forward: input must be at least 2D");
    assert(input->shape[input->ndim - 1] == l->in_features && "linear_forward: last dim of input must match in_features");
    assert(input->contiguous && "linear_forward: contiguous input");
    const int n = tensor_numel(input) / l->in_features;
    int shape[DNN_MAX_DIMS];
    for (int i = 0; i < input->ndim; i++) shape[i] = input->shape[i];
    shape[input->ndim - 1] = l->out_features;
    tensor *y = tensor_scratch(scratch, input->ndim, shape, 0);
    dnn_amd_check(dnn_hip_linear((const float *)input->data + input->offset, n, l->in_features, tensor_data_ptr(l->weight), 0,
                                 tensor_data_ptr(l->bias), l->out_features, tensor_data_ptr(y)),
                  "dnn_hip_linear");
    return y;
}

swiglu_ffn *swiglu_ffn_create(struct mem_pool *params, int d_model, int intermediate_size) {
    assert(d_model > 0 && intermediate_size > 0);
    swiglu_ffn *f = _mem_pool_alloc(params, sizeof(swiglu_ffn), NULL);
    module_init(&f->base, params, "swiglu_ffn");
    f->d_model = d_model;
    f->intermediate_size = intermediate_size;
    f->gate_proj = linear_create(params, d_model, intermediate_size);
    module_add_child(&f->base, "gate_proj", &f->gate_proj->base);
    f->up_proj = linear_create(params, d_model, intermediate_size);
    module_add_child(&f->base, "up_proj", &f->up_proj->base);
    f->down_proj = linear_create(params, intermediate_size, d_model);
    module_add_child(&f->base, "down_proj", &f->down_proj->base);
    return f;
}

rms_norm *rms_norm_create(struct mem_pool *params, int d, float eps) {
    assert(d > 0);
    rms_norm *r = _mem_pool_alloc(params, sizeof(rms_norm), NULL);
    module_init(&r->base, params, "rms_norm");
    r->d = d;
    r->eps = eps;
    r->weight = tensor_zeros(params, 1, (int[]){d}, 1);
    float *w = tensor_data_ptr(r->weight);
    for (int i = 0; i < d; i++) w[i] = 1.0f;
    module_param(&r->base, "weight", r->weight);
    return r;
}

embedding *embedding_create(struct mem_pool *params, int vocab_size, int d_model) {
    assert(vocab_size > 0 && d_model > 0);
    embedding *e = _mem_pool_alloc(params, sizeof(embedding), NULL);
    module_init(&e->base, params, "embedding");
    e->vocab_size = vocab_size;
    e->d_model = d_model;
    e->weight = tensor_uniform(params, 2, (int[]){vocab_size, d_model}, 1, 1.0f / sqrtf((float)d_model));
    module_param(&e->base, "weight", e->weight);
    return e;
}

long long linear_num_parameters(linear *l) { return module_num_parameters(&l->base); }
long long swiglu_ffn_num_parameters(swiglu_ffn *f) { return module_num_parameters(&f->base); }
long long embedding_num_parameters(embedding *e) { return module_num_parameters(&e->base); }

/* embedding_forward (nn.c:193-199 -> tensor_embedding, embedding.c:63-110):
 * the row gather runs on the device, the table resident in HBM. */
tensor *embedding_forward(struct mem_pool *scratch, struct mem_pool *data, embedding *emb, const tensor *ids) {
    (void)data;
    assert(emb && ids && ids->ndim == 1 && "embedding: ids must be 1D");
    return tensor_embedding(scratch, emb->weight, ids);
}

/* swiglu_ffn_forward (nn.c:61-78): gate and up projections, SwiGLU, down
 * projection, in one device call (weights resident after the first). */
tensor *swiglu_ffn_forward(struct mem_pool *scratch, swiglu_ffn *ffn, const tensor *x) {
    assert(ffn && x);
    assert(x->contiguous && x->ndim >= 1 && x->shape[x->ndim - 1] == ffn->d_model &&
           "swiglu_ffn_forward: x must be contiguous [..., d_model]");
    const int n = tensor_numel(x) / ffn->d_model;
    int shape[DNN_MAX_DIMS];
    for (int i = 0; i < x->ndim; i++) shape[i] = x->shape[i];
    tensor *y = tensor_scratch(scratch, x->ndim, shape, 0);
    dnn_amd_check(dnn_hip_op_swiglu_ffn((const float *)x->data + x->offset, n, ffn->d_model, ffn->intermediate_size,
                                        tensor_data_ptr(ffn->gate_proj->weight), tensor_data_ptr(ffn->gate_proj->bias),
                                        tensor_data_ptr(ffn->up_proj->weight), tensor_data_ptr(ffn->up_proj->bias),
                                        tensor_data_ptr(ffn->down_proj->weight), tensor_data_ptr(ffn->down_proj->bias),
                                        tensor_data_ptr(y)),
                  "dnn_hip_op_swiglu_ffn");
    return y;
}

/* rms_norm_forward (nn.c:169-173 -> tensor_rms_norm) on the device. */
tensor *rms_norm_forward(struct mem_pool *scratch, rms_norm *norm, const tensor *x) {
    assert(norm && x && x->contiguous && x->shape[x->ndim - 1] == norm->d);
    return tensor_rms_norm(scratch, x, norm->weight, norm->eps);
}
