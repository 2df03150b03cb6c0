/* pool.h -- bump-allocator pools.  Same struct layout and semantics as the
 * reference (include/pool.h:6-21, src/pool.c:8-57): allocation is a pointer bump,
 * _mem_pool_alloc zero-fills (or copies src), _nz leaves memory uninitialised,
 * and running out of capacity is a fatal assert. */
#ifndef DNN_POOL_H
#define DNN_POOL_H
#include <stddef.h>

typedef struct mem_pool {
    char   *buffer;
    size_t  capacity;
    size_t  offset;
} mem_pool;

mem_pool mem_pool_create(size_t capacity);
void     mem_pool_destroy(mem_pool *pool);
void     mem_pool_reset(mem_pool *pool);
size_t   mem_pool_mark(mem_pool *pool);
void     mem_pool_release(mem_pool *pool, size_t mark);
void    *_mem_pool_alloc(struct mem_pool *pool, size_t bytes, const void *src);
void    *_mem_pool_alloc_nz(struct mem_pool *pool, size_t bytes);

#endif
