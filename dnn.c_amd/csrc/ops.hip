// ops.hip -- the op-level device layer: the reference's tensor ops (ops.h,
// norm.h, rope.h, multihead.h) and its linear / SwiGLU FFN layers on host
// tensors, computed on the GPU (include/dnn_hip.h, "op level").
//
// Every call is synchronous and owns nothing of the caller's: inputs are
// copied to device buffers of a per-device context, the kernels run on its
// stream, the result is copied back.  Weight-like operands the caller marks
// as cacheable (linear / FFN weights, embedding tables: tensors of a params
// pool) stay resident in HBM, keyed by host pointer, element count and a
// sampled fingerprint, so a loop of linear_forward calls uploads each weight
// once.
//
// Numerics: the matmul and the elementwise ops are built with FP contraction
// off and sum k in order, so tensor_matmul_add (ops_matrix.c:1079-1183: sum
// over k in order, then + bias), tensor_add (ops_elem.c:110-175), tensor_rope
// (rope.c:28-32), the layout ops and the gather return the reference's NO_CBLAS
// bits exactly; tensor_swiglu uses the device's expf and tensor_rms_norm a tree
// sum of squares (within the logit tolerance of the decode path).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/dnn_hip.h"
#include "batch.h"
#include "session.h"

namespace dnnhip {
namespace {

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return set_error(DNN_HIP_EDEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

constexpr int OPS_THR = 256;
constexpr int MM_T = 64;          // output tile of the matmul: 64 x 64, 4 x 4 per thread
constexpr int MM_K = 16;          // k-slab staged in LDS per step
constexpr int MAXBATCH = DNN_HIP_VIEW_MAX_DIMS - 2;

// ---------------------------------------------------------------- kernels

struct MmArgs {
    const float *a, *b, *bias;
    float *out;
    int M, N, K;
    int a_rs, a_cs;               // a: row (M) and column (K) strides
    int b_ks, b_ns;               // b: strides along K and along N (trans_b folded in)
    int nbd;                      // batch dims
    int bshape[MAXBATCH];
    int a_bs[MAXBATCH], b_bs[MAXBATCH];   // batch strides (0 where broadcast)
};

// out[batch][m][n] = (sum_k a[m][k] * b[k][n], k in order) + bias[n]
__global__ __launch_bounds__(OPS_THR) void mm_kernel(MmArgs p) {
#pragma clang fp contract(off)
    __shared__ float As[MM_K][MM_T + 1];
    __shared__ float Bs[MM_K][MM_T + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * MM_T, n0 = blockIdx.x * MM_T;
    long long a_off = 0, b_off = 0;
    {
        int r = blockIdx.z;
        for (int d = p.nbd - 1; d >= 0; d--) {
            const int c = r % p.bshape[d];
            r /= p.bshape[d];
            a_off += (long long)c * p.a_bs[d];
            b_off += (long long)c * p.b_bs[d];
        }
    }
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.f;
    for (int k0 = 0; k0 < p.K; k0 += MM_K) {
#pragma unroll
        for (int q = 0; q < MM_T * MM_K / OPS_THR; q++) {
            const int e = tid + q * OPS_THR;
            const int am = e / MM_K, ak = e % MM_K;                 // A slab [m][k]
            const int gm = m0 + am, gk = k0 + ak;
            As[ak][am] = (gm < p.M && gk < p.K) ? p.a[a_off + (long long)gm * p.a_rs + (long long)gk * p.a_cs] : 0.f;
            const int bk = e / MM_T, bn = e % MM_T;                 // B slab [k][n]
            const int hk = k0 + bk, hn = n0 + bn;
            Bs[bk][bn] = (hk < p.K && hn < p.N) ? p.b[b_off + (long long)hk * p.b_ks + (long long)hn * p.b_ns] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < MM_K; kk++) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + av[i] * bv[j];
        }
        __syncthreads();
    }
    float *o = p.out + (long long)blockIdx.z * p.M * p.N;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + ty + 16 * i;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + tx + 16 * j;
            if (n < p.N) o[(long long)m * p.N + n] = acc[i][j] + p.bias[n];
        }
    }
}

// out[i] = f(a[.], b[.]) over an N-d index space with per-operand strides
// (stride 0 along a broadcast dimension).  OP 0: a + b; 1: SwiGLU
// (a / (1 + expf(-a))) * b (simd.h:394-397).
struct Ew2Args {
    const float *a, *b;
    float *out;
    long long n;
    int ndim;
    int shape[DNN_HIP_VIEW_MAX_DIMS];
    int sa[DNN_HIP_VIEW_MAX_DIMS], sb[DNN_HIP_VIEW_MAX_DIMS];
};

template <int OP>
__global__ __launch_bounds__(OPS_THR) void ew2_kernel(Ew2Args p) {
#pragma clang fp contract(off)
    for (long long i = (long long)blockIdx.x * OPS_THR + threadIdx.x; i < p.n; i += (long long)gridDim.x * OPS_THR) {
        long long r = i, oa = 0, ob = 0;
        for (int d = p.ndim - 1; d >= 0; d--) {
            const int c = (int)(r % p.shape[d]);
            r /= p.shape[d];
            oa += (long long)c * p.sa[d];
            ob += (long long)c * p.sb[d];
        }
        const float x = p.a[oa], y = p.b[ob];
        p.out[i] = OP == 0 ? x + y : (x / (1.0f + expf(-x))) * y;
    }
}

// In-place RoPE of x [outer][N][d] (rope.c:28-32): pair k of row n rotates by
// the table entry [n][k].
__global__ __launch_bounds__(OPS_THR) void rope_kernel(float *x, long long pairs, int N, int half, const float *cs,
                                                       const float *sn) {
#pragma clang fp contract(off)
    for (long long i = (long long)blockIdx.x * OPS_THR + threadIdx.x; i < pairs; i += (long long)gridDim.x * OPS_THR) {
        const int k = (int)(i % half);
        const int n = (int)((i / half) % N);
        const float c = cs[(long long)n * half + k], s = sn[(long long)n * half + k];
        const float e = x[2 * i], o = x[2 * i + 1];
        x[2 * i] = e * c - o * s;
        x[2 * i + 1] = e * s + o * c;
    }
}

// out[i][:] = table[ids[i]][:] (embedding.c:79-84)
__global__ __launch_bounds__(OPS_THR) void gather_kernel(const float *table, int D, const int *ids, float *out) {
    const long long src = (long long)ids[blockIdx.x] * D, dst = (long long)blockIdx.x * D;
    for (int c = threadIdx.x; c < D; c += OPS_THR) out[dst + c] = table[src + c];
}

// [B][N][P*H*dk] -> P tensors [B][H][N][dk] (multihead.c:240-263, 300-348)
__global__ __launch_bounds__(OPS_THR) void split_heads_kernel(const float *x, long long n, int N, int H, int dk, int P,
                                                              float *o0, float *o1, float *o2) {
    for (long long i = (long long)blockIdx.x * OPS_THR + threadIdx.x; i < n; i += (long long)gridDim.x * OPS_THR) {
        const int row = P * H * dk;
        const long long bn = i / row;
        const int c = (int)(i - bn * row);
        const int part = c / (H * dk), h = (c / dk) % H, j = c % dk;
        const long long b = bn / N, t = bn % N;
        float *o = part == 0 ? o0 : part == 1 ? o1 : o2;
        o[((b * H + h) * N + t) * dk + j] = x[i];
    }
}

// [B][H][N][dk] -> [B][N][H*dk] (multihead.c:199-232, 49-66)
__global__ __launch_bounds__(OPS_THR) void merge_heads_kernel(const float *x, long long n, int H, int N, int dk,
                                                              float *o) {
    for (long long i = (long long)blockIdx.x * OPS_THR + threadIdx.x; i < n; i += (long long)gridDim.x * OPS_THR) {
        const int j = (int)(i % dk);
        const long long t = (i / dk) % N, h = (i / ((long long)dk * N)) % H, b = i / ((long long)dk * N * H);
        o[((b * N + t) * H + h) * dk + j] = x[i];
    }
}

__global__ __launch_bounds__(OPS_THR) void fill_kernel(float *p, long long n, float v) {
    for (long long i = (long long)blockIdx.x * OPS_THR + threadIdx.x; i < n; i += (long long)gridDim.x * OPS_THR) p[i] = v;
}

unsigned grid_for(long long n) { return (unsigned)std::min<long long>((n + OPS_THR - 1) / OPS_THR, 65536); }

// ---------------------------------------------------------------- context

// Device buffers of one op call (a bump arena reserved up front), the
// resident weight cache, the stream.  One per device; calls serialise on its
// mutex.
struct OpCtx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
    char *arena = nullptr;
    size_t cap = 0, used = 0;
    struct Entry {
        const float *host;
        size_t n;
        uint64_t print;
        float *dev;
        uint64_t last;
    };
    std::vector<Entry> cache;
    size_t cache_bytes = 0;
    uint64_t tick = 0;
    float *ones = nullptr;
    size_t ones_n = 0;
};

constexpr size_t CACHE_LIMIT = (size_t)8 << 30;     // resident weights per device
std::mutex g_ctx_mu;
std::map<int, OpCtx *> g_ctx;

int ctx_get(OpCtx **out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    auto it = g_ctx.find(dev);
    if (it != g_ctx.end()) { *out = it->second; return DNN_HIP_OK; }
    auto *c = new OpCtx();
    c->device = dev;
    const hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return set_error(DNN_HIP_EDEVICE, "op stream: %s", hipGetErrorString(e));
    }
    g_ctx[dev] = c;
    *out = c;
    return DNN_HIP_OK;
}

size_t al(size_t bytes) { return (bytes + 255) / 256 * 256; }

int reserve(OpCtx *c, size_t bytes) {
    c->used = 0;
    if (bytes <= c->cap) return DNN_HIP_OK;
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->arena) (void)hipFree(c->arena);
    c->arena = nullptr;
    c->cap = 0;
    int rc = dalloc(&c->arena, bytes);
    if (rc) return rc;
    c->cap = bytes;
    return DNN_HIP_OK;
}

template <class T>
T *take(OpCtx *c, size_t count) {
    T *p = reinterpret_cast<T *>(c->arena + c->used);
    c->used += al(count * sizeof(T));
    return p;
}

uint64_t fingerprint(const float *p, size_t n) {
    uint64_t h = 1469598103934665603ULL;
    auto mix = [&](uint64_t v) { h = (h ^ v) * 1099511628211ULL; };
    mix((uint64_t)(uintptr_t)p);
    mix((uint64_t)n);
    const size_t ns = n < 4096 ? n : 4096;
    for (size_t k = 0; k < ns; k++) {
        uint32_t bits;
        memcpy(&bits, p + k * n / ns, 4);
        mix(bits);
    }
    return h;
}

// The device copy of a cacheable host operand of n floats (uploaded when it
// is new or its fingerprint changed; least recently used copies are dropped
// past CACHE_LIMIT).
int cached(OpCtx *c, const float *host, size_t n, const float **dev) {
    const uint64_t fp = fingerprint(host, n);
    c->tick++;
    for (auto &e : c->cache)
        if (e.host == host && e.n == n) {
            if (e.print != fp) {
                HIP_TRY(hipMemcpy(e.dev, host, n * sizeof(float), hipMemcpyHostToDevice));
                e.print = fp;
            }
            e.last = c->tick;
            *dev = e.dev;
            return DNN_HIP_OK;
        }
    while (c->cache_bytes + n * sizeof(float) > CACHE_LIMIT && !c->cache.empty()) {
        auto lru = std::min_element(c->cache.begin(), c->cache.end(),
                                    [](const OpCtx::Entry &x, const OpCtx::Entry &y) { return x.last < y.last; });
        HIP_TRY(hipStreamSynchronize(c->stream));
        (void)hipFree(lru->dev);
        c->cache_bytes -= lru->n * sizeof(float);
        c->cache.erase(lru);
    }
    float *d = nullptr;
    int rc = dalloc(&d, n);
    if (rc) return rc;
    const hipError_t e = hipMemcpy(d, host, n * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return set_error(DNN_HIP_EDEVICE, "weight upload: %s", hipGetErrorString(e));
    }
    c->cache.push_back({host, n, fp, d, c->tick});
    c->cache_bytes += n * sizeof(float);
    *dev = d;
    return DNN_HIP_OK;
}

// Elements a strided view spans from its first element (non-negative strides).
size_t view_span(const dnn_hip_view *v) {
    size_t s = 1;
    for (int d = 0; d < v->ndim; d++)
        if (v->shape[d] > 1) s += (size_t)(v->shape[d] - 1) * (size_t)v->strides[d];
    return s;
}

size_t view_numel(const dnn_hip_view *v) {
    size_t n = 1;
    for (int d = 0; d < v->ndim; d++) n *= (size_t)v->shape[d];
    return n;
}

int check_view(const dnn_hip_view *v, const char *what) {
    if (!v || !v->data || v->ndim < 1 || v->ndim > DNN_HIP_VIEW_MAX_DIMS)
        return set_error(DNN_HIP_EINVAL, "%s: bad view", what);
    for (int d = 0; d < v->ndim; d++)
        if (v->shape[d] < 1 || v->strides[d] < 0) return set_error(DNN_HIP_EINVAL, "%s: bad shape or stride", what);
    return DNN_HIP_OK;
}

// Uploads the span of a view (or finds its cached copy).
int upload_view(OpCtx *c, const dnn_hip_view *v, bool cache, const float **dev) {
    const size_t span = view_span(v);
    if (cache) return cached(c, v->data, span, dev);
    float *d = take<float>(c, span);
    HIP_TRY(hipMemcpyAsync(d, v->data, span * sizeof(float), hipMemcpyHostToDevice, c->stream));
    *dev = d;
    return DNN_HIP_OK;
}

int finish(OpCtx *c, float *host_out, const float *dev_out, size_t n) {
    if (host_out) HIP_TRY(hipMemcpyAsync(host_out, dev_out, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return DNN_HIP_OK;
}

// Enqueues out = a . b (+ bias) for device operands; shapes checked by callers.
int enqueue_mm(OpCtx *c, const float *a, const float *b, const float *bias, float *out, int M, int N, int K, int a_rs,
               int a_cs, int b_ks, int b_ns, int batch, int nbd, const int *bshape, const int *a_bs, const int *b_bs) {
    MmArgs p{};
    p.a = a; p.b = b; p.bias = bias; p.out = out;
    p.M = M; p.N = N; p.K = K;
    p.a_rs = a_rs; p.a_cs = a_cs; p.b_ks = b_ks; p.b_ns = b_ns;
    p.nbd = nbd;
    for (int d = 0; d < nbd; d++) { p.bshape[d] = bshape[d]; p.a_bs[d] = a_bs[d]; p.b_bs[d] = b_bs[d]; }
    if (batch > 65535) return set_error(DNN_HIP_EINVAL, "matmul: %d batch slices (at most 65535)", batch);
    hipLaunchKernelGGL(mm_kernel, dim3((N + MM_T - 1) / MM_T, (M + MM_T - 1) / MM_T, batch), dim3(OPS_THR), 0, c->stream, p);
    HIP_TRY(hipGetLastError());
    return DNN_HIP_OK;
}

}  // namespace
}  // namespace dnnhip

using namespace dnnhip;

extern "C" {

int dnn_hip_op_matmul_add(const dnn_hip_view *a, const dnn_hip_view *b, int trans_b, const float *bias, int cache_b,
                          float *out) {
    int rc = check_view(a, "matmul_add a");
    if (!rc) rc = check_view(b, "matmul_add b");
    if (rc) return rc;
    if (!bias || !out || a->ndim < 2 || b->ndim < 2) return set_error(DNN_HIP_EINVAL, "matmul_add: bad arguments");
    const int na = a->ndim, nb = b->ndim;
    const int K = a->shape[na - 1], M = a->shape[na - 2];
    const int N = trans_b ? b->shape[nb - 2] : b->shape[nb - 1];
    const int bk = trans_b ? b->shape[nb - 1] : b->shape[nb - 2];
    if (K != bk) return set_error(DNN_HIP_EINVAL, "matmul_add: inner dims %d and %d", K, bk);
    // batch broadcast (ops_matrix.c:1079-1090, _matmul_batch_off)
    const int abd = na - 2, bbd = nb - 2, nbd = std::max(abd, bbd);
    int bshape[MAXBATCH] = {0}, a_bs[MAXBATCH] = {0}, b_bs[MAXBATCH] = {0};
    int batch = 1;
    for (int i = 0; i < nbd; i++) {
        const int da = i < abd ? a->shape[abd - 1 - i] : 1, db = i < bbd ? b->shape[bbd - 1 - i] : 1;
        if (da != db && da != 1 && db != 1) return set_error(DNN_HIP_EINVAL, "matmul_add: batch dims %d and %d", da, db);
        const int d = nbd - 1 - i;
        bshape[d] = std::max(da, db);
        a_bs[d] = i < abd && da != 1 ? a->strides[abd - 1 - i] : 0;
        b_bs[d] = i < bbd && db != 1 ? b->strides[bbd - 1 - i] : 0;
        batch *= bshape[d];
    }
    OpCtx *c = nullptr;
    rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t n_out = (size_t)batch * M * N;
    rc = reserve(c, al(view_span(a) * 4) + (cache_b ? 0 : al(view_span(b) * 4)) + al((size_t)N * 4) + al(n_out * 4));
    const float *da = nullptr, *db = nullptr;
    if (!rc) rc = upload_view(c, a, false, &da);
    if (!rc) rc = upload_view(c, b, cache_b != 0, &db);
    if (rc) return rc;
    float *dbias = take<float>(c, N);
    HIP_TRY(hipMemcpyAsync(dbias, bias, (size_t)N * 4, hipMemcpyHostToDevice, c->stream));
    float *dout = take<float>(c, n_out);
    const int b_ks = trans_b ? b->strides[nb - 1] : b->strides[nb - 2];
    const int b_ns = trans_b ? b->strides[nb - 2] : b->strides[nb - 1];
    rc = enqueue_mm(c, da, db, dbias, dout, M, N, K, a->strides[na - 2], a->strides[na - 1], b_ks, b_ns, batch, nbd,
                    bshape, a_bs, b_bs);
    if (rc) return rc;
    return finish(c, out, dout, n_out);
}

static int ew2(int op, const dnn_hip_view *a, const dnn_hip_view *b, float *out) {
    int rc = check_view(a, "elementwise a");
    if (!rc) rc = check_view(b, "elementwise b");
    if (rc) return rc;
    if (!out) return set_error(DNN_HIP_EINVAL, "elementwise: out is NULL");
    // broadcast (broadcast.c:5-16): right-aligned, extents equal or 1
    Ew2Args p{};
    const int nd = std::max(a->ndim, b->ndim);
    p.ndim = nd;
    p.n = 1;
    for (int i = 0; i < nd; i++) {
        const int da = i < a->ndim ? a->shape[a->ndim - 1 - i] : 1, db = i < b->ndim ? b->shape[b->ndim - 1 - i] : 1;
        if (da != db && da != 1 && db != 1) return set_error(DNN_HIP_EINVAL, "elementwise: shapes %d and %d", da, db);
        const int d = nd - 1 - i;
        p.shape[d] = std::max(da, db);
        p.sa[d] = i < a->ndim && da != 1 ? a->strides[a->ndim - 1 - i] : 0;
        p.sb[d] = i < b->ndim && db != 1 ? b->strides[b->ndim - 1 - i] : 0;
        p.n *= p.shape[d];
    }
    OpCtx *c = nullptr;
    rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    rc = reserve(c, al(view_span(a) * 4) + al(view_span(b) * 4) + al((size_t)p.n * 4));
    const float *da = nullptr, *db = nullptr;
    if (!rc) rc = upload_view(c, a, false, &da);
    if (!rc) rc = upload_view(c, b, false, &db);
    if (rc) return rc;
    float *dout = take<float>(c, (size_t)p.n);
    p.a = da; p.b = db; p.out = dout;
    if (op == 0) hipLaunchKernelGGL(ew2_kernel<0>, dim3(grid_for(p.n)), dim3(OPS_THR), 0, c->stream, p);
    else hipLaunchKernelGGL(ew2_kernel<1>, dim3(grid_for(p.n)), dim3(OPS_THR), 0, c->stream, p);
    HIP_TRY(hipGetLastError());
    return finish(c, out, dout, (size_t)p.n);
}

int dnn_hip_op_add(const dnn_hip_view *a, const dnn_hip_view *b, float *out) { return ew2(0, a, b, out); }
int dnn_hip_op_swiglu(const dnn_hip_view *gate, const dnn_hip_view *up, float *out) { return ew2(1, gate, up, out); }

int dnn_hip_op_rms_norm(const float *x, int n, int d, const float *gamma, float eps, float *y) {
    if (!x || !y || n < 1 || d < 1) return set_error(DNN_HIP_EINVAL, "rms_norm: bad arguments (%d x %d)", n, d);
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t nx = (size_t)n * d;
    rc = reserve(c, 2 * al(nx * 4) + al((size_t)d * 4));
    if (rc) return rc;
    float *dx = take<float>(c, nx), *dy = take<float>(c, nx), *dg = take<float>(c, d);
    HIP_TRY(hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, c->stream));
    if (gamma) {
        HIP_TRY(hipMemcpyAsync(dg, gamma, (size_t)d * 4, hipMemcpyHostToDevice, c->stream));
    } else {
        hipLaunchKernelGGL(fill_kernel, dim3(grid_for(d)), dim3(OPS_THR), 0, c->stream, dg, (long long)d, 1.0f);
        HIP_TRY(hipGetLastError());
    }
    HIP_TRY(launch_rms_rows(dx, dg, dy, n, d, d, eps, c->stream));
    return finish(c, y, dy, nx);
}

int dnn_hip_op_rope(float *x, int outer, int N, int d, const float *cos_t, const float *sin_t) {
    if (!x || !cos_t || !sin_t || outer < 1 || N < 1 || d < 2 || d % 2)
        return set_error(DNN_HIP_EINVAL, "rope: bad arguments (%d x %d x %d)", outer, N, d);
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t nx = (size_t)outer * N * d, nt = (size_t)N * (d / 2);
    rc = reserve(c, al(nx * 4) + 2 * al(nt * 4));
    if (rc) return rc;
    float *dx = take<float>(c, nx), *dc = take<float>(c, nt), *ds = take<float>(c, nt);
    HIP_TRY(hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dc, cos_t, nt * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(ds, sin_t, nt * 4, hipMemcpyHostToDevice, c->stream));
    const long long pairs = (long long)nx / 2;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(pairs)), dim3(OPS_THR), 0, c->stream, dx, pairs, N, d / 2, dc, ds);
    HIP_TRY(hipGetLastError());
    return finish(c, x, dx, nx);
}

int dnn_hip_op_embedding(const float *table, int V, int D, int cache_table, const int *ids, int n, float *out) {
    if (!table || !ids || !out || V < 1 || D < 1 || n < 1) return set_error(DNN_HIP_EINVAL, "embedding: bad arguments");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= V) return set_error(DNN_HIP_ERANGE, "embedding: id %d at %d outside [0,%d)", ids[i], i, V);
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t nt = (size_t)V * D, no = (size_t)n * D;
    rc = reserve(c, (cache_table ? 0 : al(nt * 4)) + al((size_t)n * 4) + al(no * 4));
    if (rc) return rc;
    const float *dt = nullptr;
    if (cache_table) {
        rc = cached(c, table, nt, &dt);
        if (rc) return rc;
    } else {
        float *t = take<float>(c, nt);
        HIP_TRY(hipMemcpyAsync(t, table, nt * 4, hipMemcpyHostToDevice, c->stream));
        dt = t;
    }
    int *di = take<int>(c, n);
    float *dout = take<float>(c, no);
    HIP_TRY(hipMemcpyAsync(di, ids, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
    hipLaunchKernelGGL(gather_kernel, dim3(n), dim3(OPS_THR), 0, c->stream, dt, D, di, dout);
    HIP_TRY(hipGetLastError());
    return finish(c, out, dout, no);
}

int dnn_hip_op_split_heads(const float *x, int B, int N, int H, int dk, int parts, float *out0, float *out1,
                           float *out2) {
    if (!x || B < 1 || N < 1 || H < 1 || dk < 1 || (parts != 1 && parts != 3) || !out0 ||
        (parts == 3 && (!out1 || !out2)))
        return set_error(DNN_HIP_EINVAL, "split_heads: bad arguments");
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t n = (size_t)B * N * parts * H * dk, per = (size_t)B * H * N * dk;
    rc = reserve(c, al(n * 4) + parts * al(per * 4));
    if (rc) return rc;
    float *dx = take<float>(c, n);
    float *o[3] = {take<float>(c, per), nullptr, nullptr};
    if (parts == 3) { o[1] = take<float>(c, per); o[2] = take<float>(c, per); }
    HIP_TRY(hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, c->stream));
    hipLaunchKernelGGL(split_heads_kernel, dim3(grid_for((long long)n)), dim3(OPS_THR), 0, c->stream, dx, (long long)n, N,
                       H, dk, parts, o[0], o[1] ? o[1] : o[0], o[2] ? o[2] : o[0]);
    HIP_TRY(hipGetLastError());
    float *hout[3] = {out0, out1, out2};
    for (int p = 0; p < parts; p++)
        HIP_TRY(hipMemcpyAsync(hout[p], o[p], per * 4, hipMemcpyDeviceToHost, c->stream));
    return finish(c, nullptr, nullptr, 0);
}

int dnn_hip_op_merge_heads(const float *x, int B, int H, int N, int dk, float *out) {
    if (!x || !out || B < 1 || H < 1 || N < 1 || dk < 1) return set_error(DNN_HIP_EINVAL, "merge_heads: bad arguments");
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t n = (size_t)B * H * N * dk;
    rc = reserve(c, 2 * al(n * 4));
    if (rc) return rc;
    float *dx = take<float>(c, n), *dout = take<float>(c, n);
    HIP_TRY(hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, c->stream));
    hipLaunchKernelGGL(merge_heads_kernel, dim3(grid_for((long long)n)), dim3(OPS_THR), 0, c->stream, dx, (long long)n, H,
                       N, dk, dout);
    HIP_TRY(hipGetLastError());
    return finish(c, out, dout, n);
}

int dnn_hip_op_linear(const float *x, int n, int in, const float *w, int w_layout, const float *b, int out_f,
                      int cache_w, float *y) {
    if (!x || !w || !y || n < 1 || in < 1 || out_f < 1 || (w_layout != 0 && w_layout != 1))
        return set_error(DNN_HIP_EINVAL, "linear %d x %d -> %d (layout %d)", n, in, out_f, w_layout);
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t nx = (size_t)n * in, nw = (size_t)in * out_f, ny = (size_t)n * out_f;
    rc = reserve(c, al(nx * 4) + (cache_w ? 0 : al(nw * 4)) + al((size_t)out_f * 4) + al(ny * 4));
    if (rc) return rc;
    float *dx = take<float>(c, nx);
    HIP_TRY(hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, c->stream));
    const float *dw = nullptr;
    if (cache_w) {
        rc = cached(c, w, nw, &dw);
        if (rc) return rc;
    } else {
        float *t = take<float>(c, nw);
        HIP_TRY(hipMemcpyAsync(t, w, nw * 4, hipMemcpyHostToDevice, c->stream));
        dw = t;
    }
    float *db = take<float>(c, out_f);
    if (b) {
        HIP_TRY(hipMemcpyAsync(db, b, (size_t)out_f * 4, hipMemcpyHostToDevice, c->stream));
    } else {
        hipLaunchKernelGGL(fill_kernel, dim3(grid_for(out_f)), dim3(OPS_THR), 0, c->stream, db, (long long)out_f, 0.0f);
        HIP_TRY(hipGetLastError());
    }
    float *dy = take<float>(c, ny);
    // layout 0: W [in][out] (k stride out, n stride 1); layout 1: W [out][in]
    rc = enqueue_mm(c, dx, dw, db, dy, n, out_f, in, in, 1, w_layout ? 1 : out_f, w_layout ? in : 1, 1, 0, nullptr,
                    nullptr, nullptr);
    if (rc) return rc;
    return finish(c, y, dy, ny);
}

int dnn_hip_op_swiglu_ffn(const float *x, int n, int d_model, int d_ffn, const float *wg, const float *bg,
                          const float *wu, const float *bu, const float *wd, const float *bd, float *y) {
    if (!x || !y || !wg || !bg || !wu || !bu || !wd || !bd || n < 1 || d_model < 1 || d_ffn < 1)
        return set_error(DNN_HIP_EINVAL, "swiglu_ffn: bad arguments");
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    const size_t nx = (size_t)n * d_model, nh = (size_t)n * d_ffn;
    rc = reserve(c, 2 * al(nx * 4) + 3 * al(nh * 4) + 2 * al((size_t)d_ffn * 4) + al((size_t)d_model * 4));
    if (rc) return rc;
    const float *dwg = nullptr, *dwu = nullptr, *dwd = nullptr;
    rc = cached(c, wg, (size_t)d_model * d_ffn, &dwg);
    if (!rc) rc = cached(c, wu, (size_t)d_model * d_ffn, &dwu);
    if (!rc) rc = cached(c, wd, (size_t)d_ffn * d_model, &dwd);
    if (rc) return rc;
    float *dx = take<float>(c, nx), *dy = take<float>(c, nx);
    float *g = take<float>(c, nh), *u = take<float>(c, nh), *act = take<float>(c, nh);
    float *dbg = take<float>(c, d_ffn), *dbu = take<float>(c, d_ffn), *dbd = take<float>(c, d_model);
    HIP_TRY(hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dbg, bg, (size_t)d_ffn * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dbu, bu, (size_t)d_ffn * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dbd, bd, (size_t)d_model * 4, hipMemcpyHostToDevice, c->stream));
    // swiglu_ffn_forward (nn.c:61-78): gate and up projections, SwiGLU, down
    rc = enqueue_mm(c, dx, dwg, dbg, g, n, d_ffn, d_model, d_model, 1, d_ffn, 1, 1, 0, nullptr, nullptr, nullptr);
    if (!rc) rc = enqueue_mm(c, dx, dwu, dbu, u, n, d_ffn, d_model, d_model, 1, d_ffn, 1, 1, 0, nullptr, nullptr, nullptr);
    if (rc) return rc;
    Ew2Args p{};
    p.a = g; p.b = u; p.out = act; p.n = (long long)nh; p.ndim = 1; p.shape[0] = (int)nh; p.sa[0] = 1; p.sb[0] = 1;
    hipLaunchKernelGGL(ew2_kernel<1>, dim3(grid_for(p.n)), dim3(OPS_THR), 0, c->stream, p);
    HIP_TRY(hipGetLastError());
    rc = enqueue_mm(c, act, dwd, dbd, dy, n, d_model, d_ffn, d_ffn, 1, d_model, 1, 1, 0, nullptr, nullptr, nullptr);
    if (rc) return rc;
    return finish(c, y, dy, nx);
}

int dnn_hip_op_cache_drop(const float *host) {
    OpCtx *c = nullptr;
    int rc = ctx_get(&c);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (size_t i = 0; i < c->cache.size();) {
        if (!host || c->cache[i].host == host) {
            (void)hipFree(c->cache[i].dev);
            c->cache_bytes -= c->cache[i].n * sizeof(float);
            c->cache.erase(c->cache.begin() + (long)i);
        } else {
            i++;
        }
    }
    return DNN_HIP_OK;
}

}  // extern "C"
