/* context.h -- the three pools a caller owns (reference include/context.h:6-20). */
#ifndef DNN_CONTEXT_H
#define DNN_CONTEXT_H
#include "pool.h"

typedef struct dnn_ctx {
    mem_pool *params;   /* weights and model structs, never reset */
    mem_pool *scratch;  /* per-step intermediates */
    mem_pool *data;     /* batch data, generated ids, KV caches */
} dnn_ctx;

int  dnn_ctx_init(dnn_ctx *ctx, size_t params_sz, size_t scratch_sz, size_t data_sz);
void dnn_ctx_reset_step(dnn_ctx *ctx);
void dnn_ctx_destroy(dnn_ctx *ctx);

#endif
