/* pool.c -- bump pools and the three-pool context (reference src/pool.c:8-57,
 * src/context.c:5-35): same zero-fill / copy / no-fill semantics, same fatal
 * assert on exhaustion.  One deliberate difference: every allocation starts
 * on an 8-byte boundary.  A plain bump pointer hands the structs allocated
 * from a pool (module items, tensors) 4-byte-aligned memory after an
 * odd-length float array -- a misaligned access UBSan reports (undefined
 * behaviour, and a fault on strict-alignment targets); the cost is at most 4
 * bytes per allocation. */
#include "dnn/pool.h"
#include "dnn/context.h"
#include <assert.h>
#include <stdlib.h>
#include <string.h>

mem_pool mem_pool_create(size_t capacity) {
    mem_pool p;
    p.buffer = malloc(capacity);
    assert(p.buffer && "mem_pool_create: malloc failed");
    p.capacity = capacity;
    p.offset = 0;
    return p;
}

void mem_pool_destroy(mem_pool *pool) {
    if (!pool || !pool->buffer) return;
    free(pool->buffer);
    pool->buffer = NULL;
    pool->capacity = pool->offset = 0;
}

void   mem_pool_reset(mem_pool *pool) { pool->offset = 0; }
size_t mem_pool_mark(mem_pool *pool) { return pool->offset; }
void   mem_pool_release(mem_pool *pool, size_t mark) { pool->offset = mark; }

void *_mem_pool_alloc_nz(mem_pool *pool, size_t bytes) {
    const size_t start = (pool->offset + 7) & ~(size_t)7;
    assert(start + bytes <= pool->capacity && "_mem_pool_alloc_nz: out of memory");
    void *p = pool->buffer + start;
    pool->offset = start + bytes;
    return p;
}

void *_mem_pool_alloc(mem_pool *pool, size_t bytes, const void *src) {
    assert(((pool->offset + 7) & ~(size_t)7) + bytes <= pool->capacity && "_mem_pool_alloc: out of memory");
    void *p = _mem_pool_alloc_nz(pool, bytes);
    if (src) memcpy(p, src, bytes);
    else memset(p, 0, bytes);
    return p;
}

int dnn_ctx_init(dnn_ctx *ctx, size_t params_sz, size_t scratch_sz, size_t data_sz) {
    mem_pool *pools[3] = {malloc(sizeof(mem_pool)), malloc(sizeof(mem_pool)), malloc(sizeof(mem_pool))};
    size_t sizes[3] = {params_sz, scratch_sz, data_sz};
    int ok = pools[0] && pools[1] && pools[2];
    for (int i = 0; ok && i < 3; i++) {
        pools[i]->buffer = malloc(sizes[i]);
        pools[i]->capacity = sizes[i];
        pools[i]->offset = 0;
        if (!pools[i]->buffer) ok = 0;
    }
    if (!ok) {
        for (int i = 0; i < 3; i++)
            if (pools[i]) { free(pools[i]->buffer); free(pools[i]); }
        return -1;
    }
    ctx->params = pools[0];
    ctx->scratch = pools[1];
    ctx->data = pools[2];
    return 0;
}

void dnn_ctx_reset_step(dnn_ctx *ctx) {
    mem_pool_reset(ctx->scratch);
    mem_pool_reset(ctx->data);
}

void dnn_ctx_destroy(dnn_ctx *ctx) {
    mem_pool **ps[3] = {&ctx->params, &ctx->scratch, &ctx->data};
    for (int i = 0; i < 3; i++)
        if (*ps[i]) { mem_pool_destroy(*ps[i]); free(*ps[i]); *ps[i] = NULL; }
}
