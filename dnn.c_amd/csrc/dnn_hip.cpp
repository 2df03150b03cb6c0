// dnn_hip.cpp -- the C-ABI device layer (include/dnn_hip.h): HBM mirror of the
// parameters, KV rings, and the launch of the persistent decode kernel.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdlib>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/dnn_hip.h"
#include "decode_kernel.h"
#include "session.h"

using namespace dnnhip;

namespace {

thread_local std::string g_err;

template <class... A>
int fail(int code, const char *fmt, A... args) {
    return dnnhip::set_error(code, fmt, args...);
}

#define HIP_TRY(expr)                                                                  \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return fail(DNN_HIP_EDEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

int dnnhip::set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

namespace {

enum { P_WQKV, P_BQKV, P_WO, P_BO, P_GA, P_GF, P_WG, P_BG, P_WU, P_BU, P_WD, P_BD, NPL };

// Device layout: every tensor 256-byte aligned inside one arena.
void plan_layout(dnn_hip_model *m) {
    size_t o = 0;
    auto take = [&](size_t floats) { size_t r = o; o = round_up(o + floats * sizeof(float), 256); return r; };
    const size_t D = m->D, F = m->F, V = m->V, ldD = m->ldD, ldF = m->ldF;
    m->off.embed = take(V * ldD);
    m->off.lm_bias = take(V);
    m->off.g_final = take(ldD);
    m->off.l.assign((size_t)m->L * NPL, 0);
    for (int l = 0; l < m->L; l++) {
        size_t *p = &m->off.l[(size_t)l * NPL];
        p[P_WQKV] = take(3 * D * ldD);
        p[P_BQKV] = take(3 * D);
        p[P_WO] = take(D * ldD);
        p[P_BO] = take(D);
        p[P_GA] = take(ldD);
        p[P_GF] = take(ldD);
        p[P_WG] = take(2 * F * ldD);   // gate and up rows interleaved
        p[P_BG] = take(F);
        p[P_WU] = 0;                   // lives inside P_WG
        p[P_BU] = take(F);
        p[P_WD] = take(D * ldF);
        p[P_BD] = take(D);
    }
    m->arena_bytes = o;
}

// W [K][N] (the reference's [in][out]) -> dst[n*ld + k], zero padding k >= K.
// dst rows are spaced by row_step*ld floats (2 for the interleaved gate/up pair).
void transpose_into(float *dst, const float *W, int K, int N, int ld, int row_step) {
    const int TB = 64;
    for (int k0 = 0; k0 < K; k0 += TB)
        for (int n0 = 0; n0 < N; n0 += TB)
            for (int n = n0; n < std::min(N, n0 + TB); n++) {
                float *d = dst + (size_t)n * row_step * ld;
                for (int k = k0; k < std::min(K, k0 + TB); k++) d[k] = W[(size_t)k * N + n];
            }
}

int upload(dnn_hip_model *m, const float *const *params, int n_params) {
    const int need = 1 + NPL * m->L + 2;
    if (!params || n_params != need)
        return fail(DNN_HIP_EINVAL, "expected %d parameter pointers, got %d", need, n_params);
    for (int i = 0; i < need; i++)
        if (!params[i]) return fail(DNN_HIP_EINVAL, "parameter %d is NULL", i);
    const int D = m->D, F = m->F, V = m->V, ldD = m->ldD, ldF = m->ldF;
    std::vector<char> host(m->arena_bytes, 0);
    auto at = [&](size_t off) { return reinterpret_cast<float *>(host.data() + off); };
    for (int v = 0; v < V; v++) memcpy(at(m->off.embed) + (size_t)v * ldD, params[0] + (size_t)v * D, sizeof(float) * D);
    memcpy(at(m->off.lm_bias), params[1 + NPL * m->L + 1], sizeof(float) * V);
    memcpy(at(m->off.g_final), params[1 + NPL * m->L], sizeof(float) * D);
    for (int l = 0; l < m->L; l++) {
        const float *const *p = params + 1 + (size_t)l * NPL;
        const size_t *o = &m->off.l[(size_t)l * NPL];
        transpose_into(at(o[P_WQKV]), p[P_WQKV], D, 3 * D, ldD, 1);
        memcpy(at(o[P_BQKV]), p[P_BQKV], sizeof(float) * 3 * D);
        transpose_into(at(o[P_WO]), p[P_WO], D, D, ldD, 1);
        memcpy(at(o[P_BO]), p[P_BO], sizeof(float) * D);
        memcpy(at(o[P_GA]), p[P_GA], sizeof(float) * D);
        memcpy(at(o[P_GF]), p[P_GF], sizeof(float) * D);
        transpose_into(at(o[P_WG]), p[P_WG], D, F, ldD, 2);
        transpose_into(at(o[P_WG]) + ldD, p[P_WU], D, F, ldD, 2);
        memcpy(at(o[P_BG]), p[P_BG], sizeof(float) * F);
        memcpy(at(o[P_BU]), p[P_BU], sizeof(float) * F);
        transpose_into(at(o[P_WD]), p[P_WD], F, D, ldF, 1);
        memcpy(at(o[P_BD]), p[P_BD], sizeof(float) * D);
    }
    if (m->bf16) {
        // W16A32: every weight matrix rounded to bf16 (round to nearest even);
        // the fp32 arena keeps the rounded values too (the embedding gather and
        // the persistent kernels read it), the bf16 arena feeds the batched GEMMs
        std::vector<uint16_t> h16(m->arena_bytes / sizeof(float), 0);
        auto round_range = [&](size_t off, size_t n) {
            uint32_t *f = reinterpret_cast<uint32_t *>(host.data() + off);
            uint16_t *h = h16.data() + off / sizeof(float);
            for (size_t i = 0; i < n; i++) {
                const uint32_t u = f[i];
                const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
                h[i] = (uint16_t)r;
                f[i] = r << 16;
            }
        };
        round_range(m->off.embed, (size_t)V * ldD);
        for (int l = 0; l < m->L; l++) {
            const size_t *o = &m->off.l[(size_t)l * NPL];
            round_range(o[P_WQKV], (size_t)3 * D * ldD);
            round_range(o[P_WO], (size_t)D * ldD);
            round_range(o[P_WG], (size_t)2 * F * ldD);
            round_range(o[P_WD], (size_t)D * ldF);
        }
        HIP_TRY(hipSetDevice(m->device));
        HIP_TRY(hipMemcpy(m->arena16, h16.data(), h16.size() * sizeof(uint16_t), hipMemcpyHostToDevice));
    }
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(hipMemcpy(m->arena, host.data(), m->arena_bytes, hipMemcpyHostToDevice));
    m->packed_valid = false;                 // the batched engine repacks at its next use
    return DNN_HIP_OK;
}

void free_session_buffers(dnn_hip_session *s) {
    void *bufs[] = {s->kc, s->vc, s->xa, s->pos, s->steps_done, s->err, s->feed, s->n_feed, s->ids, s->logits};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
}

int pick_nb(int B) { return B > 4 ? 8 : B > 2 ? 4 : B > 1 ? 2 : 1; }

}  // namespace

extern "C" {

const char *dnn_hip_last_error(void) { return g_err.c_str(); }

int dnn_hip_init(int device) {
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(DNN_HIP_EINVAL, "device %d of %d", device, n);
    HIP_TRY(hipSetDevice(device));
    return dnnhip::static_scratch_setup(device);
}

int dnn_hip_model_create(int V, int D, int L, int H, int dk, int F, const float *const *params,
                         int n_params, const float *eps, dnn_hip_model **out) {
    return dnn_hip_model_create_ex(V, D, L, H, dk, F, params, n_params, eps, DNN_HIP_WEIGHTS_F32, out);
}

int dnn_hip_model_create_ex(int V, int D, int L, int H, int dk, int F, const float *const *params,
                            int n_params, const float *eps, int weights, dnn_hip_model **out) {
    if (!out) return fail(DNN_HIP_EINVAL, "out is NULL");
    if (weights != DNN_HIP_WEIGHTS_F32 && weights != DNN_HIP_WEIGHTS_BF16)
        return fail(DNN_HIP_EINVAL, "weights %d: DNN_HIP_WEIGHTS_F32 or DNN_HIP_WEIGHTS_BF16", weights);
    *out = nullptr;
    if (V <= 0 || D <= 0 || L <= 0 || H <= 0 || F <= 0 || dk <= 0)
        return fail(DNN_HIP_EINVAL, "non-positive dimension");
    if (D != H * dk) return fail(DNN_HIP_EINVAL, "d_model %d != n_heads %d * d_k %d", D, H, dk);
    if (dk != DK) return fail(DNN_HIP_EINVAL, "the decode kernels are built for d_k=%d (got %d)", DK, dk);
    if (D % 2 || V % 2) return fail(DNN_HIP_EINVAL, "d_model and vocab_size must be even");
    if (D > 3 * LDALIGN) return fail(DNN_HIP_EINVAL, "d_model %d: the decode kernels cover d_model <= %d", D, 3 * LDALIGN);
    if (F > FCMAX * LDALIGN) return fail(DNN_HIP_EINVAL, "d_ffn %d: the decode kernels cover d_ffn <= %d", F, FCMAX * LDALIGN);
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    auto *m = new dnn_hip_model();
    m->V = V; m->D = D; m->L = L; m->H = H; m->dk = dk; m->F = F;
    m->ldD = (int)round_up(D, LDALIGN);
    m->ldF = (int)round_up(F, LDALIGN);
    m->device = dev;
    m->bf16 = weights == DNN_HIP_WEIGHTS_BF16;
    m->eps.assign(2 * L + 1, 1e-5f);
    if (eps) for (int i = 0; i < 2 * L + 1; i++) m->eps[i] = eps[i];
    m->eps_final = m->eps[2 * L];
    plan_layout(m);
    // every access goes through 32-bit buffer offsets
    if (m->arena_bytes >= 0x7fffffffu) {
        const size_t bytes = m->arena_bytes;
        delete m;
        return fail(DNN_HIP_EINVAL, "weights need %zu bytes; one decode arena holds < 2 GiB", bytes);
    }
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&m->arena), m->arena_bytes);
    if (e != hipSuccess) { delete m; return fail(DNN_HIP_ENOMEM, "hipMalloc(%zu) for weights: %s", m->arena_bytes, hipGetErrorString(e)); }
    if (m->bf16) {
        e = hipMalloc(reinterpret_cast<void **>(&m->arena16), m->arena_bytes / 2);
        if (e != hipSuccess) {
            (void)hipFree(m->arena);
            delete m;
            return fail(DNN_HIP_ENOMEM, "hipMalloc(%zu) for bf16 weights: %s", m->arena_bytes / 2, hipGetErrorString(e));
        }
    }
    int rc = upload(m, params, n_params);
    if (rc != DNN_HIP_OK) { (void)hipFree(m->arena); if (m->arena16) (void)hipFree(m->arena16); delete m; return rc; }
    auto fo = [](size_t byte_off) { return (uint32_t)(byte_off / sizeof(float)); };
    std::vector<LayerOff> lo(L);
    for (int l = 0; l < L; l++) {
        const size_t *o = &m->off.l[(size_t)l * NPL];
        LayerOff &w = lo[l];
        w.wqkv = fo(o[P_WQKV]); w.bqkv = fo(o[P_BQKV]);
        w.wo = fo(o[P_WO]); w.bo = fo(o[P_BO]);
        w.g_attn = fo(o[P_GA]); w.g_ffn = fo(o[P_GF]);
        w.wgu = fo(o[P_WG]); w.bg = fo(o[P_BG]); w.bu = fo(o[P_BU]);
        w.wd = fo(o[P_WD]); w.bd = fo(o[P_BD]);
        w.eps_attn = m->eps[2 * l];
        w.eps_ffn = m->eps[2 * l + 1];
    }
    m->h_layers = lo;
    e = hipMalloc(reinterpret_cast<void **>(&m->d_layers), sizeof(LayerOff) * L);
    if (e == hipSuccess) e = hipMemcpy(m->d_layers, lo.data(), sizeof(LayerOff) * L, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(m->arena);
        if (m->d_layers) (void)hipFree(m->d_layers);
        delete m;
        return fail(DNN_HIP_EDEVICE, "layer table upload: %s", hipGetErrorString(e));
    }
    *out = m;
    return DNN_HIP_OK;
}

int dnn_hip_model_update(dnn_hip_model *m, const float *const *params, int n_params) {
    if (!m) return fail(DNN_HIP_EINVAL, "model is NULL");
    return upload(m, params, n_params);
}

int dnn_hip_model_rope(dnn_hip_model *m, const float *cos_table, const float *sin_table, int rows) {
    if (!m) return fail(DNN_HIP_EINVAL, "model is NULL");
    HIP_TRY(hipSetDevice(m->device));
    if (m->rope) { (void)hipFree(m->rope); m->rope = nullptr; }
    m->rope_rows = 0;
    if (!cos_table || !sin_table) return DNN_HIP_OK;
    if (rows <= 0) return fail(DNN_HIP_EINVAL, "rope rows %d", rows);
    const size_t n = (size_t)rows * (m->dk / 2);
    int rc = dalloc(&m->rope, 2 * n);
    if (rc) return rc;
    HIP_TRY(hipMemcpy(m->rope, cos_table, n * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(m->rope + n, sin_table, n * sizeof(float), hipMemcpyHostToDevice));
    m->rope_rows = rows;
    return DNN_HIP_OK;
}

int dnn_hip_model_destroy(dnn_hip_model *m) {
    if (!m) return DNN_HIP_OK;
    (void)hipSetDevice(m->device);
    if (m->arena) (void)hipFree(m->arena);
    if (m->arena16) (void)hipFree(m->arena16);
    if (m->packed) (void)hipFree(m->packed);
    if (m->d_layers) (void)hipFree(m->d_layers);
    if (m->rope) (void)hipFree(m->rope);
    delete m;
    return DNN_HIP_OK;
}

int dnn_hip_session_create(dnn_hip_model *m, int B, int max_seq, dnn_hip_session **out) {
    if (!m || !out) return fail(DNN_HIP_EINVAL, "NULL argument");
    *out = nullptr;
    if (B <= 0 || B > MAX_ROWS) return fail(DNN_HIP_EINVAL, "batch %d outside [1,%d]", B, MAX_ROWS);
    if (max_seq <= 0) return fail(DNN_HIP_EINVAL, "max_seq %d", max_seq);
    HIP_TRY(hipSetDevice(m->device));
    auto *s = new dnn_hip_session();
    s->m = m;
    s->B = B;
    s->max_seq = max_seq;
    s->kv_s = (int)round_up((size_t)max_seq, BK_SEQ_ALIGN);
    s->h_pos.assign(B, 0);
    if (const char *k = getenv("DNN_HIP_DECODE_KERNEL")) s->kernel_pref = atoi(k);
    if (const char *k = getenv("DNN_HIP_ATT_SPLITS")) s->att_splits_req = atoi(k);
    // the batched engine for more than 4 rows (from 5 rows on it beats the
    // persistent kernel, which runs 5-8 rows at its 8-row cost: C2 at 8 rows
    // 17.8k vs 15.4k tokens/s, 1,024-key histories 14.5k vs 11.5k), or on
    // request; DNN_HIP_DECODE_KERNEL=3 keeps up to 8 rows of an fp32 model on
    // the persistent kernel (its bf16 form covers 1-4 rows)
    s->batched = B > MAXB || s->kernel_pref == 6 || (B > 4 && (s->kernel_pref != 3 || m->bf16));
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, m->device) != hipSuccess || n_cu <= 0) n_cu = 256;
    s->grid_cap = n_cu;
    // room for heads split over up to ATT_SPLIT_MAX workgroups when B*H allows it
    s->ex = Exch{m->ldD, m->ldF, m->D, B, s->grid_cap, m->H, B * m->H <= ATT_SPLIT_HEADS ? ATT_SPLIT_MAX : 1};
    // the kernels read whole 64-key chunks: the row stride kv_s covers them
    const size_t kv = (size_t)m->L * B * m->H * s->kv_s * DK + (size_t)CH * DK;
    const size_t xa_pairs = s->batched ? 1 : s->ex.total(m->L);
    s->xa_pairs = xa_pairs;
    if (kv * sizeof(float) >= 0x7fffffffu || xa_pairs * 8 >= 0x7fffffffu) {
        delete s;
        return fail(DNN_HIP_EINVAL, "KV cache of %zu bytes per tensor / exchange of %zu bytes: each must stay < 2 GiB",
                    kv * sizeof(float), xa_pairs * 8);
    }
    int rc = 0;
    rc = rc ? rc : dalloc(&s->kc, kv);
    rc = rc ? rc : dalloc(&s->vc, kv);
    rc = rc ? rc : dalloc(&s->xa, xa_pairs);
    rc = rc ? rc : dalloc(&s->pos, (size_t)B);
    rc = rc ? rc : dalloc(&s->steps_done, 1);
    rc = rc ? rc : dalloc(&s->err, 1);
    rc = rc ? rc : dalloc(&s->n_feed, (size_t)B);
    if (rc) { free_session_buffers(s); delete s; return rc; }
    hipError_t e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&s->ev0);
    if (e == hipSuccess) e = hipEventCreate(&s->ev1);
    // tag 0 is never a step's tag, so a zeroed arena holds no valid value; its
    // padding columns stay 0.0 for ever (they meet zero weights)
    if (e == hipSuccess) e = hipMemset(s->xa, 0, sizeof(uint2) * xa_pairs);
    if (e == hipSuccess) e = hipMemset(s->kc, 0, sizeof(float) * kv);
    if (e == hipSuccess) e = hipMemset(s->vc, 0, sizeof(float) * kv);
    if (e == hipSuccess) e = hipMemset(s->pos, 0, sizeof(int) * (size_t)B);
    if (e != hipSuccess) {
        free_session_buffers(s);
        delete s;
        return fail(DNN_HIP_EDEVICE, "session setup: %s", hipGetErrorString(e));
    }
    *out = s;
    return DNN_HIP_OK;
}

int dnn_hip_session_reset(dnn_hip_session *s) {
    if (!s) return fail(DNN_HIP_EINVAL, "session is NULL");
    HIP_TRY(hipSetDevice(s->m->device));
    HIP_TRY(hipMemset(s->pos, 0, sizeof(int) * (size_t)s->B));
    std::fill(s->h_pos.begin(), s->h_pos.end(), 0);
    return DNN_HIP_OK;
}

int dnn_hip_session_lengths(dnn_hip_session *s, int *lens) {
    if (!s || !lens) return fail(DNN_HIP_EINVAL, "NULL argument");
    memcpy(lens, s->h_pos.data(), sizeof(int) * (size_t)s->B);
    return DNN_HIP_OK;
}

int dnn_hip_session_destroy(dnn_hip_session *s) {
    if (!s) return DNN_HIP_OK;
    (void)hipSetDevice(s->m->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->eng) engine_destroy(s->eng);
    free_session_buffers(s);
    if (s->ev0) (void)hipEventDestroy(s->ev0);
    if (s->ev1) (void)hipEventDestroy(s->ev1);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    if (s->stage) (void)hipHostFree(s->stage);
    delete s;
    return DNN_HIP_OK;
}

int dnn_hip_session_set_grid(dnn_hip_session *s, int n) {
    if (!s || n < 0) return fail(DNN_HIP_EINVAL, "bad argument");
    s->grid_req = n;
    return DNN_HIP_OK;
}

int dnn_hip_session_grid(dnn_hip_session *s, int *grid) {
    if (!s || !grid) return fail(DNN_HIP_EINVAL, "NULL argument");
    *grid = s->grid;
    return DNN_HIP_OK;
}

int dnn_hip_session_kernel(dnn_hip_session *s, int *which) {
    if (!s || !which) return fail(DNN_HIP_EINVAL, "NULL argument");
    *which = s->kernel_used;
    return DNN_HIP_OK;
}

int dnn_hip_session_att_splits(dnn_hip_session *s, int *splits) {
    if (!s || !splits) return fail(DNN_HIP_EINVAL, "NULL argument");
    *splits = s->att_splits;
    return DNN_HIP_OK;
}

int dnn_hip_session_last_ms(dnn_hip_session *s, float *ms) {
    if (!s || !ms) return fail(DNN_HIP_EINVAL, "NULL argument");
    *ms = s->last_ms;
    return DNN_HIP_OK;
}

extern "C++" {
// Workgroups per (row, head) of decode_v3's attention in a launch whose rows
// reach at most pmax positions: enough that each wavefront walks at most 4
// 32-key chunks (measured on the C2 shape: a split costs the out_proj
// workgroups more staging than it saves below that), records of at most a
// fifth of the grid (the attention role's share), and at most ns_cap; req > 0
// fixes it instead.
int dnnhip::att_splits_for(const dnn_hip_model *m, int B, int ns_cap, int req, int grid, int pmax) {
    const int heads = B * m->H;
    if (ns_cap <= 1) return 1;
    if (req > 0) return std::min(req, ns_cap);
    const int nch = (pmax + CH - 1) / CH;
    int ns = std::min(ns_cap, (nch + 4 * WPB - 1) / (4 * WPB));
    while (ns > 1 && heads * ns > grid / 5) ns--;     // the attention role's share of the grid
    return std::max(ns, 1);
}

int dnnhip::stage_begin(dnn_hip_session *s, size_t bytes) {
    s->stage_used = 0;
    if (bytes <= s->stage_cap) return DNN_HIP_OK;
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (s->stage) (void)hipHostFree(s->stage);
    s->stage = nullptr;
    s->stage_cap = 0;
    const size_t cap = std::max(bytes, (size_t)64 << 10);
    const hipError_t e = hipHostMalloc(reinterpret_cast<void **>(&s->stage), cap, hipHostMallocDefault);
    if (e != hipSuccess) {
        s->stage = nullptr;
        return fail(DNN_HIP_ENOMEM, "hipHostMalloc(%zu) for the staging buffer: %s", cap, hipGetErrorString(e));
    }
    s->stage_cap = cap;
    return DNN_HIP_OK;
}

int dnnhip::stage_copy(dnn_hip_session *s, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return DNN_HIP_OK;
    if (s->stage_used + stage_size(bytes) > s->stage_cap)
        return fail(DNN_HIP_EINVAL, "staging: %zu bytes past the %zu reserved", s->stage_used + bytes, s->stage_cap);
    char *p = s->stage + s->stage_used;
    memcpy(p, src, bytes);
    s->stage_used += stage_size(bytes);
    HIP_TRY(hipMemcpyAsync(dst, p, bytes, hipMemcpyHostToDevice, s->stream));
    return DNN_HIP_OK;
}

int dnnhip::stage_copy2d(dnn_hip_session *s, void *dst, size_t dpitch, const void *src, size_t spitch, size_t width,
                         size_t rows) {
    if (width == 0 || rows == 0) return DNN_HIP_OK;
    const size_t bytes = width * rows;
    if (s->stage_used + stage_size(bytes) > s->stage_cap)
        return fail(DNN_HIP_EINVAL, "staging: %zu bytes past the %zu reserved", s->stage_used + bytes, s->stage_cap);
    char *p = s->stage + s->stage_used;
    for (size_t r = 0; r < rows; r++) memcpy(p + r * width, static_cast<const char *>(src) + r * spitch, width);
    s->stage_used += stage_size(bytes);
    HIP_TRY(hipMemcpy2DAsync(dst, dpitch, p, width, width, rows, hipMemcpyHostToDevice, s->stream));
    return DNN_HIP_OK;
}

int dnnhip::check_decode(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps,
                         std::vector<int> &nf, int *nf_max) {
    dnn_hip_model *m = s->m;
    const int B = s->B;
    nf.assign(B, 0);
    *nf_max = 0;
    for (int b = 0; b < B; b++) {
        nf[b] = n_feed ? n_feed[b] : n_feed_all;
        if (nf[b] < 1) return fail(DNN_HIP_EINVAL, "row %d: n_feed %d < 1", b, nf[b]);
        *nf_max = std::max(*nf_max, nf[b]);
    }
    for (int t = 0; t < *nf_max; t++)
        for (int b = 0; b < B; b++)
            if (t < nf[b] && (feed[(size_t)t * B + b] < 0 || feed[(size_t)t * B + b] >= m->V))
                return fail(DNN_HIP_ERANGE, "token id %d at step %d row %d outside [0,%d)",
                            feed[(size_t)t * B + b], t, b, m->V);
    for (int b = 0; b < B; b++) {
        if (s->h_pos[b] + n_steps > s->max_seq)
            return fail(DNN_HIP_ERANGE, "row %d: %d cached + %d steps exceeds max_seq %d", b, s->h_pos[b], n_steps, s->max_seq);
        if (m->rope && s->h_pos[b] + n_steps > m->rope_rows)
            return fail(DNN_HIP_ERANGE, "row %d: position %d beyond the RoPE table (%d rows)", b, s->h_pos[b] + n_steps - 1, m->rope_rows);
    }
    return DNN_HIP_OK;
}
}  // extern "C++"

namespace {

// Workgroups per (row, head) of decode_v3's attention in a launch of n_steps,
// from the longest history the launch reaches (att_splits_for);
// DNN_HIP_ATT_SPLITS fixes it instead.
int att_splits(const dnn_hip_session *s, int grid, int n_steps) {
    int pmax = 0;
    for (int b = 0; b < s->B; b++) pmax = std::max(pmax, s->h_pos[b] + n_steps);
    return dnnhip::att_splits_for(s->m, s->B, s->ex.ns, s->att_splits_req, grid, pmax);
}

// Validate and enqueue one launch of a persistent decode kernel on the
// session's stream; decode_finish waits for it.
int decode_launch(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps, int eos,
                  bool want_logits) {
    dnn_hip_model *m = s->m;
    const int B = s->B;
    std::vector<int> nf;
    int nf_max = 0;
    int rc = dnnhip::check_decode(s, feed, n_feed_all, n_feed, n_steps, nf, &nf_max);
    if (rc) return rc;
    const int dc = m->ldD / LDALIGN;
    const int nb = pick_nb(B);
    HIP_TRY(hipSetDevice(m->device));
    int lds_max = 0;
    HIP_TRY(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, m->device));
    int grid = s->grid_cap;
    if (s->grid_req > 0) grid = std::min(grid, s->grid_req);
    const void *kern = decode_kernel_for(nb, dc, m->bf16 != 0);
    const size_t shmem = lds_bytes(nb, m->ldD, m->ldF);
    if (!kern) return fail(DNN_HIP_EINVAL, "d_model %d: the decode kernels cover d_model <= %d", m->D, 3 * LDALIGN);
    s->kernel_used = 3;
    rc = grow(&s->feed, &s->feed_cap, (size_t)nf_max * B);
    if (!rc) rc = grow(&s->ids, &s->ids_cap, (size_t)n_steps * B);
    if (!rc && want_logits) rc = grow(&s->logits, &s->logits_cap, (size_t)n_steps * B * m->V);
    if (rc) return rc;
    const size_t feed_bytes = sizeof(int) * (size_t)nf_max * B, nf_bytes = sizeof(int) * B;
    rc = stage_begin(s, stage_size(feed_bytes) + stage_size(nf_bytes));
    if (!rc) rc = stage_copy(s, s->feed, feed, feed_bytes);
    if (!rc) rc = stage_copy(s, s->n_feed, nf.data(), nf_bytes);
    if (rc) return rc;
    HIP_TRY(hipMemsetAsync(s->err, 0, sizeof(int), s->stream));

    // One workgroup (8 wavefronts) per CU: the dataflow waits need every
    // wavefront resident at once.  The launch is a plain one (a cooperative
    // launch would tie the global wave-sync resource to this process); every
    // wait is bounded, so a launch that could not be co-scheduled ends with an
    // error instead of hanging.
    if (shmem > (size_t)lds_max)
        return fail(DNN_HIP_EINVAL, "decode kernel needs %zu B of LDS for %d rows, the device has %d", shmem, nb, lds_max);
    HIP_TRY(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem));
    int per_cu = 0;
    HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, BLOCK, shmem));
    if (per_cu <= 0) return fail(DNN_HIP_EDEVICE, "decode kernel does not fit on a CU");
    s->grid = grid;

    DecodeArgs a{};
    a.V = m->V; a.D = m->D; a.L = m->L; a.H = m->H; a.F = m->F; a.ldD = m->ldD; a.ldF = m->ldF;
    a.wts = reinterpret_cast<const float *>(m->arena);
    a.wts_bytes = (uint32_t)m->arena_bytes;
    a.wts16 = m->bf16 ? m->arena16 : nullptr;
    a.embed = (uint32_t)(m->off.embed / sizeof(float));
    a.lm_bias = (uint32_t)(m->off.lm_bias / sizeof(float));
    a.g_final = (uint32_t)(m->off.g_final / sizeof(float));
    a.layers = m->d_layers;
    a.eps_final = m->eps_final;
    a.rope = m->rope; a.rope_rows = m->rope_rows;
    a.B = B; a.max_seq = s->kv_s;
    a.kc = s->kc; a.vc = s->vc; a.xa = s->xa; a.ex = s->ex;
    a.ex.grid = s->grid_cap;
    a.ex.ns = att_splits(s, grid, n_steps);
    s->att_splits = a.ex.ns;
    a.pos = s->pos; a.feed = s->feed; a.n_feed = s->n_feed;
    a.ids = s->ids; a.logits = want_logits ? s->logits : nullptr;
    a.n_steps = n_steps; a.eos = eos; a.step0 = s->next_tag; a.err = s->err; a.steps_done = s->steps_done;
    a.seq_limit = m->rope ? std::min(s->max_seq, m->rope_rows) : s->max_seq;
    Roles roles{};
    if (!plan_roles(grid, m->D, m->F, m->ldD, m->ldF, B * m->H * a.ex.ns, roles, hold_rounds(nb, m->ldD / LDALIGN)))
        return fail(DNN_HIP_EINVAL, "a grid of %d workgroups is too small for the decode kernel's roles", grid);
    if (const char *e = getenv("DNN_HIP_ROLES")) {     // "n_ac,n_d,n_e": a fixed split (tuning)
        Roles r{};
        if (sscanf(e, "%d,%d,%d", &r.n_ac, &r.n_d, &r.n_e) != 3 || r.n_ac < 1 || r.n_d < 1 || r.n_e < 1 ||
            r.n_ac + r.n_d + r.n_e >= grid)
            return fail(DNN_HIP_EINVAL, "DNN_HIP_ROLES=%s: needs n_ac,n_d,n_e >= 1 with a sum below the grid %d", e, grid);
        roles = r;
    }
    a.n_ac = roles.n_ac; a.n_d = roles.n_d; a.n_e = roles.n_e;
    s->next_tag += (unsigned)n_steps;
    void *kargs[] = {&a};
    HIP_TRY(hipEventRecord(s->ev0, s->stream));
    HIP_TRY(hipLaunchKernel(kern, dim3(grid), dim3(BLOCK), kargs, shmem, s->stream));
    HIP_TRY(hipEventRecord(s->ev1, s->stream));
    return DNN_HIP_OK;
}

// timed: the launch was the session's own (its events bracket it); otherwise
// the caller has synchronised the shared launch.
int decode_finish(dnn_hip_session *s, int *ids, float *logits, int *steps_done, bool timed = true) {
    dnn_hip_model *m = s->m;
    const int B = s->B;
    if (timed) {
        HIP_TRY(hipEventSynchronize(s->ev1));
        HIP_TRY(hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1));
    }
    int done = 0, kerr = 0;
    HIP_TRY(hipMemcpy(&kerr, s->err, sizeof(int), hipMemcpyDeviceToHost));
    if (kerr) return fail(DNN_HIP_EDEVICE, "decode kernel: a dependency wait timed out (error bits %#x); results discarded", kerr);
    HIP_TRY(hipMemcpy(&done, s->steps_done, sizeof(int), hipMemcpyDeviceToHost));
    if (ids) HIP_TRY(hipMemcpy(ids, s->ids, sizeof(int) * (size_t)done * B, hipMemcpyDeviceToHost));
    if (logits) HIP_TRY(hipMemcpy(logits, s->logits, sizeof(float) * (size_t)done * B * m->V, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(s->h_pos.data(), s->pos, sizeof(int) * B, hipMemcpyDeviceToHost));
    if (steps_done) *steps_done = done;
    return DNN_HIP_OK;
}

int decode_finish_launch(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps, int eos,
                         int *ids, float *logits, int *steps_done) {
    const int rc = decode_launch(s, feed, n_feed_all, n_feed, n_steps, eos, logits != nullptr);
    return rc ? rc : decode_finish(s, ids, logits, steps_done);
}

}  // namespace

int dnn_hip_decode(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed,
                   int n_steps, int eos, int *ids, float *logits, int *steps_done) {
    if (!s || !feed) return fail(DNN_HIP_EINVAL, "NULL argument");
    if (n_steps <= 0) return fail(DNN_HIP_EINVAL, "n_steps %d", n_steps);
    if (s->batched) return engine_decode(s, feed, n_feed_all, n_feed, n_steps, eos, ids, logits, steps_done);
    return decode_finish_launch(s, feed, n_feed_all, n_feed, n_steps, eos, ids, logits, steps_done);
}

int dnn_hip_prefill(dnn_hip_session *s, const float *embeds, int n_embed, const int *ids, int n_ids_max,
                    const int *n_ids, int mode, int prefix_len, int *next_ids, float *logits) {
    if (!s || !next_ids) return fail(DNN_HIP_EINVAL, "NULL argument");
    return engine_prefill(s, embeds, n_embed, ids, n_ids_max, n_ids, mode, prefix_len, next_ids, logits);
}

int dnn_hip_block_forward(dnn_hip_session *s, int layer, const float *x, int n_new, int pos0, int mode,
                          int prefix_len, float *y) {
    if (!s) return fail(DNN_HIP_EINVAL, "session is NULL");
    return engine_block(s, layer, x, n_new, pos0, mode, prefix_len, y);
}

int dnn_hip_head_forward(dnn_hip_session *s, const float *x, int n, int norm, float *logits) {
    if (!s) return fail(DNN_HIP_EINVAL, "session is NULL");
    return engine_head(s, x, n, norm, logits);
}

int dnn_hip_embed(dnn_hip_session *s, const int *ids, int n, float *out) {
    if (!s) return fail(DNN_HIP_EINVAL, "session is NULL");
    return engine_embed(s, ids, n, out);
}

int dnn_hip_rms_norm(dnn_hip_session *s, const float *x, const float *gamma, int n, int d, float eps, float *y) {
    if (!s) return fail(DNN_HIP_EINVAL, "session is NULL");
    return engine_rms_norm(s, x, gamma, n, d, eps, y);
}

int dnn_hip_linear(const float *x, int n, int in, const float *w, int w_layout, const float *b, int out, float *y) {
    return dnn_hip_op_linear(x, n, in, w, w_layout, b, out, 1, y);
}

int dnn_hip_cache_read(dnn_hip_session *s, int layer, int which, int len, float *out) {
    if (!s || !out) return fail(DNN_HIP_EINVAL, "NULL argument");
    dnn_hip_model *m = s->m;
    if (layer < 0 || layer >= m->L || (which != 0 && which != 1) || len < 0 || len > s->max_seq)
        return fail(DNN_HIP_EINVAL, "layer %d / which %d / len %d", layer, which, len);
    HIP_TRY(hipSetDevice(m->device));
    const size_t per = (size_t)m->H * DK * s->kv_s;           // floats per (layer, row)
    std::vector<float> h((size_t)s->B * per);
    const float *src = (which == 0 ? s->kc : s->vc) + (size_t)layer * s->B * per;
    HIP_TRY(hipStreamSynchronize(s->stream));
    HIP_TRY(hipMemcpy(h.data(), src, h.size() * sizeof(float), hipMemcpyDeviceToHost));
    for (int b = 0; b < s->B; b++)
        for (int hh = 0; hh < m->H; hh++) {
            const float *hd = h.data() + ((size_t)b * m->H + hh) * DK * s->kv_s;
            float *o = out + (((size_t)b * m->H + hh) * len) * DK;
            for (int p = 0; p < len; p++)
                for (int d = 0; d < DK; d++)
                    o[(size_t)p * DK + d] = which == 0 ? hd[(size_t)d * s->kv_s + p] : hd[(size_t)p * DK + d];
        }
    return DNN_HIP_OK;
}

int dnn_hip_generate(dnn_hip_model *m, const int *prompt, int P, int max_new, int eos, int *out, int *n_out) {
    if (!m || !prompt || !out || !n_out) return fail(DNN_HIP_EINVAL, "NULL argument");
    if (P <= 0 || max_new <= 0) return fail(DNN_HIP_EINVAL, "prompt %d / max_new %d", P, max_new);
    dnn_hip_session *s = nullptr;
    int rc = dnn_hip_session_create(m, 1, P + max_new, &s);
    if (rc) return rc;
    const int steps = P + max_new - 1;
    std::vector<int> ids(steps);
    int done = 0;
    rc = dnn_hip_decode(s, prompt, P, nullptr, steps, eos, ids.data(), nullptr, &done);
    dnn_hip_session_destroy(s);
    if (rc) return rc;
    if (out != prompt) memmove(out, prompt, sizeof(int) * P);
    int n = P;
    for (int t = P - 1; t < done; t++) {
        out[n++] = ids[t];
        if (eos >= 0 && ids[t] == eos) break;
    }
    *n_out = n;
    return DNN_HIP_OK;
}

}  // extern "C"
