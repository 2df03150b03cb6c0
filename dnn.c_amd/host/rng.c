/* rng.c -- xorshift128+ / SplitMix64 / Box-Muller, the reference's streams
 * (src/rng.c:6-78), so dnn_seed(s) + decoder_lm_create give identical weights. */
#include "dnn/rng.h"
#include <math.h>

static uint64_t next_u64(dnn_rng *r) {
    uint64_t a = r->s[0], b = r->s[1];
    r->s[0] = b;
    a ^= a << 23;
    r->s[1] = a ^ b ^ (a >> 18) ^ (b >> 5);
    return r->s[1] + b;
}

static uint64_t mix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ULL;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
    return x ^ (x >> 31);
}

dnn_rng dnn_rng_seed(uint64_t seed) {
    dnn_rng r;
    r.s[0] = mix64(seed);
    r.s[1] = mix64(r.s[0]);
    return r;
}

float dnn_rng_uniform(dnn_rng *r) { return (float)(next_u64(r) >> 11) * 0x1.0p-53f; }

float dnn_rng_normal(dnn_rng *r) {
    float u1;
    do { u1 = dnn_rng_uniform(r); } while (u1 == 0.0f);
    float u2 = dnn_rng_uniform(r);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

int dnn_rng_uniform_int(dnn_rng *r, int n) {
    if (n <= 1) return 0;
    uint32_t limit = (uint32_t)n, mask = limit;
    for (int sh = 1; sh <= 16; sh <<= 1) mask |= mask >> sh;
    uint32_t v;
    do { v = (uint32_t)(next_u64(r) >> 32) & mask; } while (v >= limit);
    return (int)v;
}

static _Thread_local dnn_rng g_default = {{1, 2}};
dnn_rng *dnn_get_rng(void) { return &g_default; }
void dnn_seed(uint64_t seed) { g_default = dnn_rng_seed(seed); }
