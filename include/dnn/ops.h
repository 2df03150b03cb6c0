/* ops.h -- the reference's tensor ops on the decode path (reference
 * include/ops.h:7-63), computed on the device through dnn_hip.h's op level.
 * Inputs are host tensors (any strides; offsets honoured), outputs new
 * contiguous tensors in the scratch pool, as in the reference.  Forward only:
 * no autograd tape is recorded (training is not part of this library). */
#ifndef DNN_OPS_H
#define DNN_OPS_H
#include "tensor.h"

/* a + b with right-aligned broadcasting (ops.h:7, ops_elem.c:110-175); the
 * reference's bits. */
tensor *tensor_add(struct mem_pool *scratch, const tensor *a, const tensor *b);

/* (a @ b) + bias, or (a @ b^T) + bias with trans_b (ops.h:21,
 * ops_matrix.c:964-1183): a [..., M, K], b [..., K, N] or [..., N, K], batch
 * dimensions broadcast, bias [N] required.  The sum runs over k in order and
 * the bias is added last, without FMA contraction: the reference's NO_CBLAS
 * bits.  A b that requires grad (a parameter) stays resident in HBM. */
tensor *tensor_matmul_add(struct mem_pool *scratch, const tensor *a,
                          const tensor *b, int trans_b, const tensor *bias);

/* (g / (1 + expf(-g))) * u, broadcast as tensor_add (ops.h:29,
 * ops_activation.c:283-333).  The device's expf: within the logit tolerance,
 * not the reference's bits. */
tensor *tensor_swiglu(struct mem_pool *scratch, const tensor *gate, const tensor *up);

/* Rows of table [V, D] (contiguous) for ids [N] int32 -> [N, D] (ops.h:63,
 * embedding.c:63-110); an id outside [0, V) asserts.  A table that requires
 * grad (a parameter) stays resident in HBM. */
tensor *tensor_embedding(struct mem_pool *scratch, const tensor *table, const tensor *ids);

/* a ++ b along dim (ops.h:78, ops_elem.c:903-945); declared in tensor.h too. */
tensor *tensor_cat(struct mem_pool *scratch, const tensor *a, const tensor *b, int dim);

#endif
