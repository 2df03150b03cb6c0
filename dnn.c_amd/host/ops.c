/* ops.c -- the reference's tensor ops (ops.h, norm.h, rope.h, multihead.h) on
 * host tensors, computed on the device through dnn_hip.h's op level.  Shapes,
 * asserts and output allocation follow the reference (ops_elem.c:110-175,
 * ops_matrix.c:964-1183, ops_activation.c:283-333, embedding.c:63-110,
 * norm.c:404-495, rope.c:92-144, multihead.c:199-348); no autograd tape is
 * recorded. */
#include "dnn/ops.h"
#include "dnn/norm.h"
#include "dnn/rope.h"
#include "dnn/multihead.h"
#include "dnn_hip.h"
#include "device.h"
#include <assert.h>
#include <string.h>

static dnn_hip_view view_of(const tensor *t) {
    dnn_hip_view v;
    memset(&v, 0, sizeof v);
    v.data = (const float *)t->data + t->offset;
    v.ndim = t->ndim;
    for (int d = 0; d < t->ndim; d++) {
        v.shape[d] = t->shape[d];
        v.strides[d] = t->strides[d];
    }
    return v;
}

/* right-aligned broadcast shape (broadcast.c:5-16); 0 if incompatible */
static int bcast_shape(const tensor *a, const tensor *b, int *shape) {
    const int nd = a->ndim > b->ndim ? a->ndim : b->ndim;
    for (int i = 0; i < nd; i++) {
        const int da = i < a->ndim ? a->shape[a->ndim - 1 - i] : 1;
        const int db = i < b->ndim ? b->shape[b->ndim - 1 - i] : 1;
        if (da != db && da != 1 && db != 1) return 0;
        shape[nd - 1 - i] = da > db ? da : db;
    }
    return nd;
}

tensor *tensor_add(struct mem_pool *scratch, const tensor *a, const tensor *b) {
    assert(a && b);
    int shape[DNN_MAX_DIMS];
    const int nd = bcast_shape(a, b, shape);
    assert(nd > 0 && "tensor_add: incompatible shapes");
    tensor *out = tensor_scratch(scratch, nd, shape, 0);
    const dnn_hip_view va = view_of(a), vb = view_of(b);
    dnn_amd_check(dnn_hip_op_add(&va, &vb, tensor_data_ptr(out)), "dnn_hip_op_add");
    return out;
}

tensor *tensor_swiglu(struct mem_pool *scratch, const tensor *gate, const tensor *up) {
    assert(gate && up);
    int shape[DNN_MAX_DIMS];
    const int nd = bcast_shape(gate, up, shape);
    assert(nd > 0 && "tensor_swiglu: incompatible shapes");
    tensor *out = tensor_scratch(scratch, nd, shape, 0);
    const dnn_hip_view vg = view_of(gate), vu = view_of(up);
    dnn_amd_check(dnn_hip_op_swiglu(&vg, &vu, tensor_data_ptr(out)), "dnn_hip_op_swiglu");
    return out;
}

tensor *tensor_matmul_add(struct mem_pool *scratch, const tensor *a, const tensor *b, int trans_b, const tensor *bias) {
    assert(a && b && bias);
    assert(a->ndim >= 2 && b->ndim >= 2 && "tensor_matmul_add: need at least 2D");
    assert(bias->ndim == 1 && "tensor_matmul_add: bias must be 1-D");
    const int na = a->ndim, nb = b->ndim;
    const int K = a->shape[na - 1], M = a->shape[na - 2];
    const int N = trans_b ? b->shape[nb - 2] : b->shape[nb - 1];
    const int b_inner = trans_b ? b->shape[nb - 1] : b->shape[nb - 2];
    assert(K == b_inner && "tensor_matmul_add: inner dim mismatch");
    assert(bias->shape[0] == N && "tensor_matmul_add: bias size != out cols");
    int shape[DNN_MAX_DIMS];
    int nd = 2;
    if (na > 2 || nb > 2) {
        /* batch dimensions broadcast (ops_matrix.c:1079-1090) */
        const int abd = na - 2, bbd = nb - 2, nbd = abd > bbd ? abd : bbd;
        for (int i = 0; i < nbd; i++) {
            const int da = i < abd ? a->shape[abd - 1 - i] : 1, db = i < bbd ? b->shape[bbd - 1 - i] : 1;
            assert((da == db || da == 1 || db == 1) && "tensor_matmul_add: batch dims");
            shape[nbd - 1 - i] = da > db ? da : db;
        }
        nd = nbd + 2;
    }
    shape[nd - 2] = M;
    shape[nd - 1] = N;
    tensor *out = tensor_scratch(scratch, nd, shape, 0);
    const dnn_hip_view va = view_of(a), vb = view_of(b);
    float *bd = (float *)bias->data + bias->offset;
    assert(bias->ndim == 1 && (bias->strides[0] == 1 || N == 1) && "tensor_matmul_add: bias must be contiguous");
    dnn_amd_check(dnn_hip_op_matmul_add(&va, &vb, trans_b, bd, tensor_requires_grad(b), tensor_data_ptr(out)),
                  "dnn_hip_op_matmul_add");
    return out;
}

tensor *tensor_embedding(struct mem_pool *scratch, const tensor *table, const tensor *ids) {
    assert(table && ids);
    assert(table->ndim == 2 && "embedding: table must be 2D");
    assert(ids->ndim == 1 && "embedding: ids must be 1D");
    assert(table->contiguous && "embedding: table must be contiguous");
    const int V = table->shape[0], D = table->shape[1], N = ids->shape[0];
    const int *id = (const int *)ids->data + ids->offset;
    for (int i = 0; i < N; i++) assert(id[(size_t)i * ids->strides[0]] >= 0 && id[(size_t)i * ids->strides[0]] < V &&
                                       "embedding: id out of range");
    tensor *out = tensor_scratch(scratch, 2, (int[]){N, D}, 0);
    int *dense = NULL;
    if (ids->strides[0] != 1) {
        dense = (int *)_mem_pool_alloc_nz(scratch, sizeof(int) * (size_t)N);
        for (int i = 0; i < N; i++) dense[i] = id[(size_t)i * ids->strides[0]];
        id = dense;
    }
    dnn_amd_check(dnn_hip_op_embedding((const float *)table->data + table->offset, V, D, tensor_requires_grad(table),
                                       id, N, tensor_data_ptr(out)),
                  "dnn_hip_op_embedding");
    return out;
}

tensor *tensor_rms_norm(struct mem_pool *scratch, const tensor *x, const tensor *weight, float eps) {
    assert(x);
    assert(tensor_is_contiguous(x) && "tensor_rms_norm: x must be contiguous");
    const int d = x->shape[x->ndim - 1], n = tensor_numel(x) / d;
    if (weight) assert(tensor_numel(weight) == d && tensor_is_contiguous(weight));
    tensor *out = tensor_scratch(scratch, x->ndim, x->shape, 0);
    dnn_amd_check(dnn_hip_op_rms_norm((const float *)x->data + x->offset, n, d,
                                      weight ? (const float *)weight->data + weight->offset : NULL, eps,
                                      tensor_data_ptr(out)),
                  "dnn_hip_op_rms_norm");
    return out;
}

tensor *tensor_rope(struct mem_pool *scratch, tensor *x, const tensor *freqs_cos, const tensor *freqs_sin) {
    assert(x);
    assert(freqs_cos && freqs_sin);
    assert(tensor_is_contiguous(x) && "tensor_rope: x must be contiguous");
    assert(tensor_is_contiguous(freqs_cos) && "tensor_rope: freqs_cos must be contiguous");
    assert(tensor_is_contiguous(freqs_sin) && "tensor_rope: freqs_sin must be contiguous");
    assert(x->ndim >= 2 && "tensor_rope: x must have at least 2 dims");
    const int d = x->shape[x->ndim - 1], N = x->shape[x->ndim - 2];
    assert(d % 2 == 0 && "tensor_rope: last dim must be even");
    assert(freqs_cos->ndim == 2 && freqs_cos->shape[0] == N && freqs_cos->shape[1] == d / 2);
    assert(freqs_sin->ndim == 2 && freqs_sin->shape[0] == N && freqs_sin->shape[1] == d / 2);
    const int outer = tensor_numel(x) / (N * d);
    dnn_amd_check(dnn_hip_op_rope((float *)x->data + x->offset, outer, N, d,
                                  (const float *)freqs_cos->data + freqs_cos->offset,
                                  (const float *)freqs_sin->data + freqs_sin->offset),
                  "dnn_hip_op_rope");
    /* a tensor sharing x's buffer (rope.c:124-133) */
    tensor *out = _mem_pool_alloc(scratch, sizeof(tensor), x);
    out->parent = NULL;
    out->grad_fn = NULL;
    out->grad = NULL;
    return out;
}

tensor *tensor_split_heads(struct mem_pool *scratch, tensor *t, int H) {
    assert(t->ndim == 3 && "split_heads: input must be 3D [B, N, H*d_k]");
    assert(t->contiguous && "split_heads: input must be contiguous");
    const int B = t->shape[0], N = t->shape[1], D = t->shape[2];
    assert(H > 0 && D % H == 0 && "split_heads: D must be H*d_k");
    const int dk = D / H;
    tensor *out = tensor_scratch(scratch, 4, (int[]){B, H, N, dk}, 0);
    dnn_amd_check(dnn_hip_op_split_heads((const float *)t->data + t->offset, B, N, H, dk, 1, tensor_data_ptr(out), NULL,
                                         NULL),
                  "dnn_hip_op_split_heads");
    return out;
}

tensor *tensor_merge_heads(struct mem_pool *scratch, tensor *t) {
    assert(t->ndim == 4 && "merge_heads: input must be 4D [B, H, N, d_k]");
    const int B = t->shape[0], H = t->shape[1], N = t->shape[2], dk = t->shape[3];
    tensor *out = tensor_scratch(scratch, 3, (int[]){B, N, H * dk}, 0);
    dnn_amd_check(dnn_hip_op_merge_heads((const float *)t->data + t->offset, B, H, N, dk, tensor_data_ptr(out)),
                  "dnn_hip_op_merge_heads");
    return out;
}

void tensor_split_qkv_heads(struct mem_pool *scratch, tensor *qkv, int H, tensor **Qh_out, tensor **Kh_out,
                            tensor **Vh_out) {
    assert(qkv->ndim == 3 && "split_qkv_heads: qkv must be 3D [B,N,3*H*d_k]");
    assert(qkv->contiguous && "split_qkv_heads: qkv must be contiguous");
    const int B = qkv->shape[0], N = qkv->shape[1], D = qkv->shape[2];
    assert(H > 0 && D % (3 * H) == 0 && "split_qkv_heads: D must be 3*H*d_k");
    const int dk = D / (3 * H);
    const int shape4[] = {B, H, N, dk};
    tensor *Qh = tensor_scratch(scratch, 4, shape4, 0);
    tensor *Kh = tensor_scratch(scratch, 4, shape4, 0);
    tensor *Vh = tensor_scratch(scratch, 4, shape4, 0);
    dnn_amd_check(dnn_hip_op_split_heads((const float *)qkv->data + qkv->offset, B, N, H, dk, 3, tensor_data_ptr(Qh),
                                         tensor_data_ptr(Kh), tensor_data_ptr(Vh)),
                  "dnn_hip_op_split_heads");
    *Qh_out = Qh;
    *Kh_out = Kh;
    *Vh_out = Vh;
}
