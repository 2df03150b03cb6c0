/* rope.h -- RoPE tables (reference include/rope.h, src/rope.c:148-171):
 * theta_k = powf(base, -2k/dim), cos/sin(n * theta_k), [max_seq_len][dim/2]. */
#ifndef DNN_ROPE_H
#define DNN_ROPE_H
#include "tensor.h"

void tensor_rope_freqs_init(struct mem_pool *params, tensor **freqs_cos, tensor **freqs_sin,
                            int dim, int max_seq_len, float base);

#endif
