/* norm.h -- RMS normalisation (reference include/norm.h:35), on the device. */
#ifndef DNN_NORM_H
#define DNN_NORM_H
#include "tensor.h"

/* y = x * rsqrt(mean(x^2) + eps) * weight over the last dimension of a
 * contiguous x (norm.c:404-495); weight [d] or NULL (treated as 1).  Returns
 * a new scratch tensor of x's shape.  Forward only. */
tensor *tensor_rms_norm(struct mem_pool *scratch, const tensor *x,
                        const tensor *weight, float eps);

#endif
