/* module.h -- parameter registry (reference include/module.h:17-109): the same
 * structs, depth-first registration order, and the "DNNM" v1 state-dict format. */
#ifndef DNN_MODULE_H
#define DNN_MODULE_H
#include "tensor.h"

typedef enum module_item_kind { MODULE_ITEM_PARAM = 1, MODULE_ITEM_CHILD = 2 } module_item_kind;

typedef struct module_item {
    struct module_item *next;
    module_item_kind    kind;
    const char         *name;
    union { tensor *param; struct module *child; } as;
} module_item;

typedef struct module {
    struct mem_pool *pool;
    const char      *type_name;
    struct module   *parent;
    module_item     *items_head;
    module_item     *items_tail;
    int              n_items;
    int              n_direct_params;
    int              n_children;
    tensor         **flat_params;
    int              n_flat;
} module;

void      module_init(module *m, struct mem_pool *pool, const char *type_name);
void      module_param(module *m, const char *name, tensor *t);
void      module_add_child(module *m, const char *name, module *child);
tensor  **module_parameters(module *m, int *n_out);
long long module_num_parameters(module *m);
tensor   *module_find_param(module *m, const char *name);

#define MODULE_STATE_MAX_NAME 4096
void module_save(module *m, const char *path);
void module_load(module *m, const char *path, int strict);

#endif
