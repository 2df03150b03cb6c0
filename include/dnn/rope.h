/* rope.h -- rotary position embedding (reference include/rope.h:27-49):
 * tables theta_k = powf(base, -2k/dim), cos/sin(n * theta_k), [max_seq_len][dim/2]
 * (rope.c:148-171), and the rotation itself, on the device. */
#ifndef DNN_ROPE_H
#define DNN_ROPE_H
#include "tensor.h"

/* Rotates x [..., N, d] (contiguous) in place, pair k of row n by
 * freqs_cos/freqs_sin [N, d/2] (rope.h:27, rope.c:92-144): e' = e*c - o*s,
 * o' = e*s + o*c.  Returns a tensor sharing x's buffer.  The reference's bits.
 * Forward only. */
tensor *tensor_rope(struct mem_pool *scratch,
                    tensor *x, const tensor *freqs_cos, const tensor *freqs_sin);

void tensor_rope_freqs_init(struct mem_pool *params, tensor **freqs_cos, tensor **freqs_sin,
                            int dim, int max_seq_len, float base);

#endif
