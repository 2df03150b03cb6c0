/* rope.c -- RoPE frequency tables (reference src/rope.c:148-171): the same libm
 * calls in the same order, so the device gets the reference's table bits. */
#include "dnn/rope.h"
#include <assert.h>
#include <math.h>

void tensor_rope_freqs_init(struct mem_pool *params, tensor **freqs_cos, tensor **freqs_sin,
                            int dim, int max_seq_len, float base) {
    assert(dim > 0 && dim % 2 == 0 && "dim must be positive and even");
    assert(max_seq_len > 0);
    if (base == 0.0f) base = 10000.0f;
    const int half = dim / 2;
    *freqs_cos = tensor_zeros(params, 2, (int[]){max_seq_len, half}, 0);
    *freqs_sin = tensor_zeros(params, 2, (int[]){max_seq_len, half}, 0);
    float *c = (*freqs_cos)->data, *s = (*freqs_sin)->data;
    for (int k = 0; k < half; k++) {
        const float theta = powf(base, -2.0f * k / (float)dim);
        for (int n = 0; n < max_seq_len; n++) {
            const float angle = (float)n * theta;
            c[n * half + k] = cosf(angle);
            s[n * half + k] = sinf(angle);
        }
    }
}
