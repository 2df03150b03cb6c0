/* tensor.c -- tensor creation and views (reference src/tensor.c:98-399), for the
 * no-grad generation path: views never record autograd state here. */
#include "dnn/tensor.h"
#include "dnn/rng.h"
#include <assert.h>
#include <string.h>

static int count(const int *shape, int ndim) {
    int n = 1;
    for (int i = 0; i < ndim; i++) n *= shape[i];
    return n;
}

static void packed_strides(int ndim, const int *shape, int *strides) {
    int s = 1;
    for (int d = ndim - 1; d >= 0; d--) { strides[d] = s; s *= shape[d]; }
}

static int is_packed(const int *shape, const int *strides, int ndim) {
    int s = 1;
    for (int d = ndim - 1; d >= 0; d--) {
        if (strides[d] != s) return 0;
        s *= shape[d];
    }
    return 1;
}

/* struct first, then zeroed (or uninitialised, fill=0) data, as tensor.c:98-132 */
static tensor *make(struct mem_pool *pool, int ndim, const int *shape, int requires_grad, int fill) {
    assert(pool && ndim > 0 && ndim <= DNN_MAX_DIMS);
    tensor *t = _mem_pool_alloc(pool, sizeof(tensor), NULL);
    t->ndim = ndim;
    memcpy(t->shape, shape, sizeof(int) * (size_t)ndim);
    packed_strides(ndim, shape, t->strides);
    size_t bytes = (size_t)count(shape, ndim) * sizeof(float);
    t->data = fill ? _mem_pool_alloc(pool, bytes, NULL) : _mem_pool_alloc_nz(pool, bytes);
    t->pool = pool;
    t->requires_grad = requires_grad ? 1 : 0;
    t->contiguous = 1;
    return t;
}

tensor *tensor_zeros(struct mem_pool *pool, int ndim, const int *shape, int requires_grad) {
    return make(pool, ndim, shape, requires_grad, 1);
}

tensor *tensor_zeros_data(struct mem_pool *pool, int ndim, const int *shape) {
    return make(pool, ndim, shape, 0, 1);
}

tensor *tensor_scratch(struct mem_pool *pool, int ndim, const int *shape, int requires_grad) {
    return make(pool, ndim, shape, requires_grad, 0);
}

tensor *tensor_randn(struct mem_pool *pool, int ndim, const int *shape, int requires_grad) {
    tensor *t = make(pool, ndim, shape, requires_grad, 1);
    float *p = t->data;
    for (int i = 0, n = count(shape, ndim); i < n; i++) p[i] = dnn_rng_normal(dnn_get_rng());
    return t;
}

/* (2u - 1) * bound, u from the default stream (tensor.c:154-162) */
tensor *tensor_uniform(struct mem_pool *pool, int ndim, const int *shape, int requires_grad, float bound) {
    tensor *t = make(pool, ndim, shape, requires_grad, 1);
    float *p = t->data;
    for (int i = 0, n = count(shape, ndim); i < n; i++)
        p[i] = (2.0f * dnn_rng_uniform(dnn_get_rng()) - 1.0f) * bound;
    return t;
}

tensor *tensor_slice(struct mem_pool *scratch, tensor *t, int dim, int start, int len) {
    assert(dim < t->ndim && start >= 0 && start + len <= t->shape[dim]);
    tensor *v = _mem_pool_alloc(scratch, sizeof(tensor), t);
    v->shape[dim] = len;
    v->offset = t->offset + start * t->strides[dim];
    v->parent = t;
    v->grad_fn = NULL;
    v->grad = NULL;
    v->pool = NULL;
    v->requires_grad = 0;
    v->contiguous = is_packed(v->shape, v->strides, v->ndim);
    return v;
}

tensor *tensor_reshape(struct mem_pool *scratch, tensor *t, int ndim, const int *shape) {
    assert(ndim > 0 && ndim <= DNN_MAX_DIMS);
    assert(tensor_is_contiguous(t) && "tensor_reshape: only contiguous tensors are reshaped here");
    int dims[DNN_MAX_DIMS], infer = -1, known = 1, total = tensor_numel(t);
    for (int i = 0; i < ndim; i++) {
        dims[i] = shape[i];
        if (shape[i] == -1) { assert(infer < 0 && "only one -1 allowed"); infer = i; }
        else { assert(shape[i] > 0); known *= shape[i]; }
    }
    if (infer >= 0) { assert(total % known == 0); dims[infer] = total / known; }
    else assert(known == total && "shape must match numel");
    tensor *v = _mem_pool_alloc(scratch, sizeof(tensor), t);
    v->ndim = ndim;
    memcpy(v->shape, dims, sizeof(int) * (size_t)ndim);
    packed_strides(ndim, dims, v->strides);
    v->parent = t;
    v->contiguous = 1;
    v->grad_fn = NULL;
    v->grad = NULL;
    v->pool = NULL;
    v->requires_grad = 0;
    return v;
}

tensor *tensor_flatten(struct mem_pool *scratch, tensor *t) {
    return tensor_reshape(scratch, t, 1, (int[]){-1});
}

/* Copies every element of src (any strides) into the packed out tensor at
 * offset `at` along dim. */
static void cat_part(float *out, const int *oshape, int ndim, int dim, int at, const tensor *src) {
    int idx[DNN_MAX_DIMS] = {0};
    const int n = count(src->shape, ndim);
    const float *sd = (const float *)src->data;
    for (int i = 0; i < n; i++) {
        size_t so = (size_t)src->offset, oo = 0;
        for (int d = 0; d < ndim; d++) {
            so += (size_t)idx[d] * src->strides[d];
            oo = oo * oshape[d] + (size_t)(idx[d] + (d == dim ? at : 0));
        }
        out[oo] = sd[so];
        for (int d = ndim - 1; d >= 0; d--) {
            if (++idx[d] < src->shape[d]) break;
            idx[d] = 0;
        }
    }
}

tensor *tensor_cat(struct mem_pool *scratch, const tensor *a, const tensor *b, int dim) {
    assert(a && b && a->ndim == b->ndim && "tensor_cat: ndim must match");
    const int ndim = a->ndim;
    if (dim < 0) dim += ndim;
    assert(dim >= 0 && dim < ndim && "tensor_cat: dim out of range");
    int shape[DNN_MAX_DIMS];
    for (int d = 0; d < ndim; d++) {
        assert((d == dim || a->shape[d] == b->shape[d]) && "tensor_cat: shape mismatch");
        shape[d] = a->shape[d];
    }
    shape[dim] += b->shape[dim];
    tensor *out = tensor_scratch(scratch, ndim, shape, 0);
    cat_part((float *)out->data, shape, ndim, dim, 0, a);
    cat_part((float *)out->data, shape, ndim, dim, a->shape[dim], b);
    return out;
}

float *tensor_data_ptr(tensor *t) {
    assert(tensor_is_contiguous(t));
    return (float *)t->data + t->offset;
}
int tensor_numel(const tensor *t) { return count(t->shape, t->ndim); }
int tensor_ndim(const tensor *t) { return t->ndim; }
int tensor_shape(const tensor *t, int dim) { return t->shape[dim]; }
int tensor_is_contiguous(const tensor *t) { return t->contiguous; }
int tensor_requires_grad(const tensor *t) { return t->requires_grad; }
