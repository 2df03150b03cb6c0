/* rng.h -- xorshift128+ with SplitMix64 seeding (reference include/rng.h:12-34,
 * src/rng.c): the same streams, so seeded weights and prompts match the
 * reference bit for bit. */
#ifndef DNN_RNG_H
#define DNN_RNG_H
#include <stdint.h>
#include <stddef.h>

typedef struct dnn_rng { uint64_t s[2]; } dnn_rng;

dnn_rng  dnn_rng_seed(uint64_t seed);
float    dnn_rng_uniform(dnn_rng *rng);
float    dnn_rng_normal(dnn_rng *rng);
int      dnn_rng_uniform_int(dnn_rng *rng, int n);
dnn_rng *dnn_get_rng(void);
void     dnn_seed(uint64_t seed);

#endif
