/* module.c -- parameter registry and the "DNNM" v1 state dict.
 *
 * Registration keeps one singly linked list of items per module; parameters
 * are discovered depth-first in registration order with duplicates dropped
 * (reference src/module.c:71-142).  That order is part of the contract: it is
 * the order weights draw from the RNG and the order dnn_hip_model_create takes.
 *
 * DNNM v1 (reference include/module.h:94-109, src/module.c:174-339), all u32
 * little-endian: "DNNM", version 1, header size 16, entry count, then per
 * entry: name length incl. NUL, name ("blocks.0.qkv_proj.weight"), ndim,
 * shape[ndim] (i32), numel, numel f32 values. */
#include "dnn/module.h"
#include <assert.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void module_init(module *m, struct mem_pool *pool, const char *type_name) {
    assert(m && pool && type_name);
    memset(m, 0, sizeof(*m));
    m->pool = pool;
    m->type_name = type_name;
}

static void no_cache_up(module *m) {
    for (; m; m = m->parent) assert(!m->flat_params && "module: registration after introspection");
}

static void push_item(module *m, module_item_kind kind, const char *name) {
    module_item *it = _mem_pool_alloc(m->pool, sizeof(module_item), NULL);
    it->kind = kind;
    it->name = name;
    if (m->items_tail) m->items_tail->next = it;
    else m->items_head = it;
    m->items_tail = it;
    m->n_items++;
}

void module_param(module *m, const char *name, tensor *t) {
    assert(m && name && t);
    assert(t->pool == m->pool && "param must live in the module's params pool");
    assert(t->parent == NULL && "registered params must not be views");
    assert(tensor_is_contiguous(t) && "registered params must be contiguous");
    no_cache_up(m);
    push_item(m, MODULE_ITEM_PARAM, name);
    m->items_tail->as.param = t;
    m->n_direct_params++;
}

void module_add_child(module *m, const char *name, module *child) {
    assert(m && name && child && child != m);
    assert(child->pool == m->pool && "child must use the same params pool");
    assert(child->parent == NULL && "child already has a parent");
    no_cache_up(m);
    push_item(m, MODULE_ITEM_CHILD, name);
    m->items_tail->as.child = child;
    m->n_children++;
    child->parent = m;
}

static int upper_bound(const module *m) {
    int n = m->n_direct_params;
    for (const module_item *it = m->items_head; it; it = it->next)
        if (it->kind == MODULE_ITEM_CHILD) n += upper_bound(it->as.child);
    return n;
}

static int collect(const module *m, tensor **out, int n) {
    for (const module_item *it = m->items_head; it; it = it->next) {
        if (it->kind == MODULE_ITEM_CHILD) { n = collect(it->as.child, out, n); continue; }
        int dup = 0;
        for (int i = 0; i < n && !dup; i++) dup = out[i] == it->as.param;
        if (!dup) out[n++] = it->as.param;
    }
    return n;
}

tensor **module_parameters(module *m, int *n_out) {
    assert(m && n_out);
    if (!m->flat_params) {
        int cap = upper_bound(m);
        m->flat_params = _mem_pool_alloc(m->pool, sizeof(tensor *) * (size_t)(cap ? cap : 1), NULL);
        m->n_flat = collect(m, m->flat_params, 0);
    }
    *n_out = m->n_flat;
    return m->flat_params;
}

long long module_num_parameters(module *m) {
    int n;
    tensor **ps = module_parameters(m, &n);
    long long total = 0;
    for (int i = 0; i < n; i++) total += tensor_numel(ps[i]);
    return total;
}

/* Visits every registered parameter with its dotted path. */
typedef int (*param_visit)(const char *path, tensor *t, void *ctx);

static int walk(module *m, char *path, size_t len, param_visit fn, void *ctx) {
    for (module_item *it = m->items_head; it; it = it->next) {
        int w = snprintf(path + len, MODULE_STATE_MAX_NAME - len,
                         it->kind == MODULE_ITEM_PARAM ? "%s" : "%s.", it->name);
        assert(w > 0 && len + (size_t)w < MODULE_STATE_MAX_NAME && "module: name too long");
        int stop = it->kind == MODULE_ITEM_PARAM ? fn(path, it->as.param, ctx)
                                                 : walk(it->as.child, path, len + (size_t)w, fn, ctx);
        path[len] = '\0';
        if (stop) return stop;
    }
    return 0;
}

typedef struct { const char *target; tensor *hit; int index, seen; } find_ctx;

static int find_visit(const char *path, tensor *t, void *vctx) {
    find_ctx *c = vctx;
    if (strcmp(path, c->target) == 0) { c->hit = t; c->index = c->seen; return 1; }
    c->seen++;
    return 0;
}

static tensor *find_indexed(module *m, const char *name, int *index) {
    char path[MODULE_STATE_MAX_NAME] = "";
    find_ctx c = {name, NULL, -1, 0};
    walk(m, path, 0, find_visit, &c);
    if (index) *index = c.index;
    return c.hit;
}

tensor *module_find_param(module *m, const char *name) { return find_indexed(m, name, NULL); }

static int count_visit(const char *path, tensor *t, void *ctx) { (void)path; (void)t; (*(int *)ctx)++; return 0; }

static void put_u32(FILE *f, uint32_t v) { fwrite(&v, 4, 1, f); }

static int save_visit(const char *path, tensor *t, void *ctx) {
    FILE *f = ctx;
    put_u32(f, (uint32_t)strlen(path) + 1);
    fwrite(path, 1, strlen(path) + 1, f);
    put_u32(f, (uint32_t)t->ndim);
    for (int d = 0; d < t->ndim; d++) { int32_t s = t->shape[d]; fwrite(&s, 4, 1, f); }
    put_u32(f, (uint32_t)tensor_numel(t));
    fwrite(tensor_data_ptr(t), sizeof(float), (size_t)tensor_numel(t), f);
    return 0;
}

void module_save(module *m, const char *path) {
    assert(m && path);
    FILE *f = fopen(path, "wb");
    assert(f && "module_save: cannot open file");
    char name[MODULE_STATE_MAX_NAME] = "";
    int n = 0;
    walk(m, name, 0, count_visit, &n);
    fwrite("DNNM", 1, 4, f);
    put_u32(f, 1);
    put_u32(f, 16);
    put_u32(f, (uint32_t)n);
    walk(m, name, 0, save_visit, f);
    fclose(f);
}

static uint32_t get_u32(FILE *f) {
    uint32_t v;
    size_t r = fread(&v, 4, 1, f);
    assert(r == 1 && "module_load: truncated file");
    (void)r;
    return v;
}

void module_load(module *m, const char *path, int strict) {
    assert(m && path);
    FILE *f = fopen(path, "rb");
    assert(f && "module_load: cannot open file");
    char magic[4];
    size_t r = fread(magic, 1, 4, f);
    assert(r == 4 && memcmp(magic, "DNNM", 4) == 0 && "module_load: bad magic");
    (void)r;
    /* read into locals first: the asserts must not hold the reads (-DNDEBUG) */
    const uint32_t version = get_u32(f);
    const uint32_t header_size = get_u32(f);
    assert(version == 1 && "module_load: unsupported version");
    assert(header_size == 16 && "module_load: unexpected header size");
    (void)version;
    (void)header_size;
    uint32_t entries = get_u32(f);
    char name[MODULE_STATE_MAX_NAME] = "";
    int live = 0;
    walk(m, name, 0, count_visit, &live);
    unsigned char *seen = strict ? calloc((size_t)live + 1, 1) : NULL;
    for (uint32_t e = 0; e < entries; e++) {
        uint32_t name_len = get_u32(f);
        assert(name_len > 0 && name_len < MODULE_STATE_MAX_NAME);
        r = fread(name, 1, name_len, f);
        assert(r == name_len && name[name_len - 1] == '\0' && "module_load: truncated file");
        uint32_t ndim = get_u32(f);
        assert(ndim > 0 && ndim <= DNN_MAX_DIMS);
        int32_t shape[DNN_MAX_DIMS];
        uint32_t prod = 1;
        for (uint32_t d = 0; d < ndim; d++) {
            shape[d] = (int32_t)get_u32(f);
            assert(shape[d] > 0);
            prod *= (uint32_t)shape[d];
        }
        uint32_t numel = get_u32(f);
        assert(numel == prod);
        int index = -1;
        tensor *t = find_indexed(m, name, &index);
        if (!t) {
            assert(!strict && "module_load: unknown param");
            fseek(f, (long)numel * (long)sizeof(float), SEEK_CUR);
            continue;
        }
        assert((uint32_t)t->ndim == ndim && "module_load: ndim mismatch");
        for (uint32_t d = 0; d < ndim; d++) assert(t->shape[d] == shape[d] && "module_load: shape mismatch");
        r = fread(tensor_data_ptr(t), sizeof(float), numel, f);
        assert(r == numel && "module_load: truncated file");
        if (seen) seen[index] = 1;
    }
    if (seen) {
        for (int i = 0; i < live; i++) assert(seen[i] && "module_load: missing live param in checkpoint");
        free(seen);
    }
    fclose(f);
}
