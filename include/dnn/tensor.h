/* tensor.h -- the reference's tensor struct (include/tensor.h:9-21), byte for
 * byte, and the subset of its functions the decode path and its callers use. */
#ifndef DNN_TENSOR_H
#define DNN_TENSOR_H
#define DNN_MAX_DIMS 8
#include "pool.h"
typedef struct grad_fn grad_fn;

typedef struct tensor {
    void    *data;
    float   *grad;
    int      shape[DNN_MAX_DIMS];
    int      strides[DNN_MAX_DIMS];
    int      ndim;
    unsigned int requires_grad : 1;
    unsigned int contiguous : 1;
    int      offset;
    struct tensor *parent;
    grad_fn *grad_fn;
    struct mem_pool *pool;
} tensor;

tensor *tensor_zeros(struct mem_pool *pool, int ndim, const int *shape, int requires_grad);
tensor *tensor_zeros_data(struct mem_pool *pool, int ndim, const int *shape);
tensor *tensor_randn(struct mem_pool *pool, int ndim, const int *shape, int requires_grad);
tensor *tensor_uniform(struct mem_pool *pool, int ndim, const int *shape, int requires_grad, float bound);
tensor *tensor_scratch(struct mem_pool *pool, int ndim, const int *shape, int requires_grad);
tensor *tensor_slice(struct mem_pool *scratch, tensor *t, int dim, int start, int len);
tensor *tensor_reshape(struct mem_pool *scratch, tensor *t, int ndim, const int *shape);
tensor *tensor_flatten(struct mem_pool *scratch, tensor *t);
/* a ++ b along dim (the other extents equal): a new contiguous scratch tensor
 * (ops_elem.c:903-945, forward only). */
tensor *tensor_cat(struct mem_pool *scratch, const tensor *a, const tensor *b, int dim);
float  *tensor_data_ptr(tensor *t);
int     tensor_numel(const tensor *t);
int     tensor_ndim(const tensor *t);
int     tensor_shape(const tensor *t, int dim);
int     tensor_is_contiguous(const tensor *t);
int     tensor_requires_grad(const tensor *t);

#endif
