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

using namespace dnnhip;

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                  \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return fail(DNN_HIP_EDEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

struct dnn_hip_model {
    int V, D, L, H, dk, F, ldD, ldF;
    int device;
    char *arena = nullptr;
    size_t arena_bytes = 0;
    LayerOff *d_layers = nullptr;    // [L] float offsets of each block's tensors
    float eps_final = 1e-5f;
    std::vector<float> eps;          // 2L+1
    float *rope = nullptr;           // [2][rope_rows][dk/2]: cos, then sin
    int rope_rows = 0;
    // byte offsets of every device tensor inside the arena, for the uploads
    struct Off { size_t embed, lm_bias, g_final; std::vector<size_t> l; } off;
};

struct dnn_hip_session {
    dnn_hip_model *m;
    int B, max_seq;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    float *kc = nullptr, *vc = nullptr;       // K^T [L][B][H][DK][max_seq], V [L][B][H][max_seq][DK]
    uint2 *xa = nullptr;                      // exchange arena (tagged pairs)
    Exch ex{};
    int *pos = nullptr, *steps_done = nullptr, *err = nullptr;
    int *feed = nullptr, *n_feed = nullptr, *ids = nullptr;
    size_t feed_cap = 0, ids_cap = 0;
    float *logits = nullptr;
    size_t logits_cap = 0;
    int grid_req = 0, grid = 0, grid_cap = 0;
    unsigned next_tag = 1;                    // tags only grow: stale values never match
    int kernel_pref = 0;                      // env DNN_HIP_DECODE_KERNEL: 4 / 5: the lookahead / streaming kernel where it applies
    int kernel_used = 0;                      // 3, 4 or 5: the kernel of the last launch
    size_t xa_pairs = 0;
    float last_ms = 0.f;
    std::vector<int> h_pos;
    // more than MAXB rows: consecutive groups of at most MAXB rows, each its own
    // session, run one after another by dnn_hip_decode
    std::vector<dnn_hip_session *> groups;
};

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
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(hipMemcpy(m->arena, host.data(), m->arena_bytes, hipMemcpyHostToDevice));
    return DNN_HIP_OK;
}

void free_session_buffers(dnn_hip_session *s) {
    void *bufs[] = {s->kc, s->vc, s->xa, s->pos, s->steps_done, s->err, s->feed, s->n_feed, s->ids, s->logits};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
}

template <class T>
int dalloc(T **p, size_t count) {
    hipError_t e = hipMalloc(reinterpret_cast<void **>(p), std::max<size_t>(count, 1) * sizeof(T));
    if (e != hipSuccess) { *p = nullptr; return fail(DNN_HIP_ENOMEM, "hipMalloc(%zu bytes): %s", count * sizeof(T), hipGetErrorString(e)); }
    return DNN_HIP_OK;
}

template <class T>
int grow(T **p, size_t *cap, size_t count) {
    if (count <= *cap) return DNN_HIP_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    int rc = dalloc(p, count);
    if (rc == DNN_HIP_OK) *cap = count;
    return rc;
}

int pick_nb(int B) { return B > 4 ? 8 : B > 2 ? 4 : B > 1 ? 2 : 1; }

// The streaming kernel's launch shape for this model, batch and grid, or
// false where it does not apply (the general kernel runs instead): every GEMV
// workgroup must own out_proj and down rows (so each takes part in every
// layer), a workgroup's biases of a phase must fit one 64-lane gather (32
// gate + 32 up for gate/up), the attention partials one 64-lane merge, and
// the weight ring must hold any one phase of a workgroup.
bool stream_plan(const dnn_hip_model *m, int B, int grid, int lds_max, StreamArgs *sa) {
    if (B > 2) return false;
    const int nb = B, NS = stream_splits(nb), NA = B * m->H * NS, NG = grid - NA;
    if (NG < 1 || NG > m->D || NA > S_MAXREC) return false;
    const int DC = m->ldD / LDALIGN, FC = m->ldF / LDALIGN;
    const int nu[5] = {3 * m->D / 2, m->D, m->F, m->D, m->V};
    const int R[5] = {2, 1, 2, 1, 1};
    const int ch[5] = {DC, DC, DC, FC, DC};
    const int bias_cap[5] = {WAVE / 2, WAVE, WAVE / 2, WAVE, WAVE};
    const int out_per_unit[4] = {2, 1, 1, 1};
    int sout = 0, ring_need = 0;
    for (int k = 0; k < 5; k++) {
        const int n_wg = (nu[k] + NG - 1) / NG;
        if (n_wg > bias_cap[k]) return false;
        ring_need = std::max(ring_need, n_wg * R[k] * ch[k]);
        if (k < 4) sout = std::max(sout, nb * n_wg * out_per_unit[k]);
    }
    const int fixed = lds5_layout(nb, m->ldD, m->ldF, m->L, sout, 0).total;
    const int rs = (lds_max - fixed) / S_SLOT;
    if (rs < ring_need) return false;
    sa->lds = lds5_layout(nb, m->ldD, m->ldF, m->L, sout, rs);
    if (sa->lds.total > lds_max) return false;
    sa->ex = Exch5{m->D, m->F, B, m->H, NS, NG};
    sa->ng = NG;
    return true;
}

}  // namespace

extern "C" {

const char *dnn_hip_last_error(void) { return g_err.c_str(); }

int dnn_hip_init(int device) {
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(DNN_HIP_EINVAL, "device %d of %d", device, n);
    HIP_TRY(hipSetDevice(device));
    return DNN_HIP_OK;
}

int dnn_hip_model_create(int V, int D, int L, int H, int dk, int F, const float *const *params,
                         int n_params, const float *eps, dnn_hip_model **out) {
    if (!out) return fail(DNN_HIP_EINVAL, "out is NULL");
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
    int rc = upload(m, params, n_params);
    if (rc != DNN_HIP_OK) { (void)hipFree(m->arena); delete m; return rc; }
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
    if (B > MAXB) {
        auto *s = new dnn_hip_session();
        s->m = m;
        s->B = B;
        s->max_seq = max_seq;
        for (int r0 = 0; r0 < B; r0 += MAXB) {
            dnn_hip_session *g = nullptr;
            const int rc = dnn_hip_session_create(m, std::min(MAXB, B - r0), max_seq, &g);
            if (rc) { dnn_hip_session_destroy(s); return rc; }
            s->groups.push_back(g);
        }
        *out = s;
        return DNN_HIP_OK;
    }
    auto *s = new dnn_hip_session();
    s->m = m;
    s->B = B;
    s->max_seq = max_seq;
    s->h_pos.assign(B, 0);
    if (const char *k = getenv("DNN_HIP_DECODE_KERNEL")) s->kernel_pref = atoi(k);   // "4": lookahead kernel
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, m->device) != hipSuccess || n_cu <= 0) n_cu = 256;
    s->grid_cap = n_cu;
    s->ex = Exch{m->ldD, m->ldF, m->D, B, s->grid_cap};
    // + CH*DK floats of zeroed padding: attention reads whole 32-key chunks,
    // and the rows past max_seq of the last head must stay inside the allocation
    const size_t kv = (size_t)m->L * B * m->H * max_seq * DK + (size_t)CH * DK;
    size_t xa_pairs = s->ex.total(m->L);
    if (B <= 2) {
        // room for the streaming kernel's exchange layout (its grid <= grid_cap)
        const int nb = pick_nb(B);
        const Exch5 e5{m->D, m->F, B, m->H, stream_splits(nb), s->grid_cap};
        xa_pairs = std::max(xa_pairs, e5.total(m->L));
    }
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
    for (dnn_hip_session *g : s->groups) {
        const int rc = dnn_hip_session_reset(g);
        if (rc) return rc;
    }
    if (!s->groups.empty()) return DNN_HIP_OK;
    HIP_TRY(hipSetDevice(s->m->device));
    HIP_TRY(hipMemset(s->pos, 0, sizeof(int) * (size_t)s->B));
    std::fill(s->h_pos.begin(), s->h_pos.end(), 0);
    return DNN_HIP_OK;
}

int dnn_hip_session_lengths(dnn_hip_session *s, int *lens) {
    if (!s || !lens) return fail(DNN_HIP_EINVAL, "NULL argument");
    if (!s->groups.empty()) {
        int r0 = 0;
        for (dnn_hip_session *g : s->groups) {
            dnn_hip_session_lengths(g, lens + r0);
            r0 += g->B;
        }
        return DNN_HIP_OK;
    }
    memcpy(lens, s->h_pos.data(), sizeof(int) * (size_t)s->B);
    return DNN_HIP_OK;
}

int dnn_hip_session_destroy(dnn_hip_session *s) {
    if (!s) return DNN_HIP_OK;
    for (dnn_hip_session *g : s->groups) dnn_hip_session_destroy(g);
    (void)hipSetDevice(s->m->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    free_session_buffers(s);
    if (s->ev0) (void)hipEventDestroy(s->ev0);
    if (s->ev1) (void)hipEventDestroy(s->ev1);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return DNN_HIP_OK;
}

int dnn_hip_session_set_grid(dnn_hip_session *s, int n) {
    if (!s || n < 0) return fail(DNN_HIP_EINVAL, "bad argument");
    for (dnn_hip_session *g : s->groups) g->grid_req = n;
    s->grid_req = n;
    return DNN_HIP_OK;
}

int dnn_hip_session_grid(dnn_hip_session *s, int *grid) {
    if (!s || !grid) return fail(DNN_HIP_EINVAL, "NULL argument");
    *grid = s->groups.empty() ? s->grid : s->groups[0]->grid;
    return DNN_HIP_OK;
}

int dnn_hip_session_kernel(dnn_hip_session *s, int *which) {
    if (!s || !which) return fail(DNN_HIP_EINVAL, "NULL argument");
    *which = s->groups.empty() ? s->kernel_used : s->groups[0]->kernel_used;
    return DNN_HIP_OK;
}

int dnn_hip_session_last_ms(dnn_hip_session *s, float *ms) {
    if (!s || !ms) return fail(DNN_HIP_EINVAL, "NULL argument");
    *ms = s->last_ms;
    return DNN_HIP_OK;
}

namespace {

// Validate and enqueue one launch of a session of at most MAXB rows on its
// stream (grid capped at grid_limit when > 0); decode_finish waits for it.
// check_only: validate the arguments, enqueue nothing.  prep: the session is
// one group of a multi-group launch: upload its inputs, fill *prep with its
// kernel arguments (general kernel, MAXB-row build) and launch nothing.
int decode_launch(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps, int eos,
                  bool want_logits, int grid_limit, bool check_only = false, DecodeArgs *prep = nullptr) {
    dnn_hip_model *m = s->m;
    const int B = s->B;
    std::vector<int> nf(B);
    int nf_max = 0;
    for (int b = 0; b < B; b++) {
        nf[b] = n_feed ? n_feed[b] : n_feed_all;
        if (nf[b] < 1) return fail(DNN_HIP_EINVAL, "row %d: n_feed %d < 1", b, nf[b]);
        nf_max = std::max(nf_max, nf[b]);
    }
    for (int t = 0; t < nf_max; t++)
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
    if (check_only) return DNN_HIP_OK;
    const int dc = m->ldD / LDALIGN;
    const int nb = prep ? MAXB : pick_nb(B);
    HIP_TRY(hipSetDevice(m->device));
    int lds_max = 0;
    HIP_TRY(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, m->device));
    int grid = s->grid_cap;
    if (s->grid_req > 0) grid = std::min(grid, s->grid_req);
    if (grid_limit > 0) grid = std::min(grid, grid_limit);
    // decode_v3 by default; the lookahead kernel (one or two rows) on request,
    // when its schedule fits (every GEMV round in at most 3 slots of the grid's
    // non-attention workgroups) and its LDS does.
    const void *kern = nullptr;
    size_t shmem = 0;
    StreamArgs sa{};
    bool stream = false;
    if (prep) {
        kern = decode_multi_for(dc);
        shmem = lds_bytes(nb, m->ldD, m->ldF);
    } else if (s->kernel_pref == 5 && stream_plan(m, B, grid, lds_max, &sa) &&
        sa.ex.total(m->L) <= s->xa_pairs) {
        kern = decode_stream_for(nb, dc);
        shmem = (size_t)sa.lds.total;
        stream = kern != nullptr;
    }
    const int rounds = (m->D + 6) / 7 + (3 * m->D / 2 + 6) / 7 + (m->D / 2 + 6) / 7 + (m->F + 6) / 7;
    if (!kern && !prep && nb <= 2 && s->kernel_pref == 4 && grid > B * m->H && rounds <= 3 * (grid - B * m->H) &&
        lds4_bytes(nb, m->ldD, m->ldF, m->L) <= (size_t)lds_max) {
        kern = decode_lookahead_for(nb, dc);
        shmem = lds4_bytes(nb, m->ldD, m->ldF, m->L);
    }
    if (!kern) {
        kern = decode_kernel_for(nb, dc);
        shmem = lds_bytes(nb, m->ldD, m->ldF);
    }
    if (!kern) return fail(DNN_HIP_EINVAL, "d_model %d: the decode kernels cover d_model <= %d", m->D, 3 * LDALIGN);
    s->kernel_used = stream ? 5 : (prep || kern == decode_kernel_for(nb, dc)) ? 3 : 4;
    int rc = grow(&s->feed, &s->feed_cap, (size_t)nf_max * B);
    if (!rc) rc = grow(&s->ids, &s->ids_cap, (size_t)n_steps * B);
    if (!rc && want_logits) rc = grow(&s->logits, &s->logits_cap, (size_t)n_steps * B * m->V);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(s->feed, feed, sizeof(int) * (size_t)nf_max * B, hipMemcpyHostToDevice, s->stream));
    HIP_TRY(hipMemcpyAsync(s->n_feed, nf.data(), sizeof(int) * B, hipMemcpyHostToDevice, s->stream));
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
    a.embed = (uint32_t)(m->off.embed / sizeof(float));
    a.lm_bias = (uint32_t)(m->off.lm_bias / sizeof(float));
    a.g_final = (uint32_t)(m->off.g_final / sizeof(float));
    a.layers = m->d_layers;
    a.eps_final = m->eps_final;
    a.rope = m->rope; a.rope_rows = m->rope_rows;
    a.B = B; a.max_seq = s->max_seq;
    a.kc = s->kc; a.vc = s->vc; a.xa = s->xa; a.ex = s->ex;
    a.ex.grid = s->grid_cap;
    a.pos = s->pos; a.feed = s->feed; a.n_feed = s->n_feed;
    a.ids = s->ids; a.logits = want_logits ? s->logits : nullptr;
    a.n_steps = n_steps; a.eos = eos; a.step0 = s->next_tag; a.err = s->err; a.steps_done = s->steps_done;
    s->next_tag += (unsigned)n_steps;
    if (prep) {
        *prep = a;
        HIP_TRY(hipStreamSynchronize(s->stream));   // inputs in place before the shared launch
        return DNN_HIP_OK;
    }
    sa.a = a;
    void *kargs[] = {stream ? static_cast<void *>(&sa) : static_cast<void *>(&a)};
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
    const int rc = decode_launch(s, feed, n_feed_all, n_feed, n_steps, eos, logits != nullptr, 0);
    return rc ? rc : decode_finish(s, ids, logits, steps_done);
}

// A session of more than MAXB rows: its groups of at most MAXB rows decode in
// one launch of the general kernel, the grid split evenly between them
// (persistent launches on separate streams are not co-resident on this
// device, so a launch per group would run them in turn); the columns of feed /
// ids / logits are gathered and scattered per group.  With eos >= 0 a group
// that stops early is run on (greedy, no stop) to the step where the last
// group stopped, so every row advances the same number of steps, as in one
// launch.
int decode_groups(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps, int eos,
                  int *ids, float *logits, int *steps_done) {
    const int B = s->B, V = s->m->V, NGR = (int)s->groups.size();
    int nf_max = 0;
    for (int b = 0; b < B; b++) nf_max = std::max(nf_max, n_feed ? n_feed[b] : n_feed_all);
    std::vector<std::vector<int>> gfeed(NGR), gnf(NGR), gids(NGR);
    std::vector<std::vector<float>> glog(NGR);
    std::vector<int> r0(NGR), done(NGR, 0), more(NGR, 0);
    for (int gi = 0, r = 0; gi < NGR; gi++) { r0[gi] = r; r += s->groups[gi]->B; }
    dnn_hip_session *lead = s->groups[0];
    dnn_hip_model *m = s->m;
    float ms = 0.f;
    // pass 0: every group from its feed; pass 1: groups that stopped early, run on
    for (int pass = 0; pass < 2; pass++) {
        if (pass == 1) {
            const int all_done = *std::max_element(done.begin(), done.end());
            for (int gi = 0; gi < NGR; gi++) more[gi] = all_done - done[gi];
        }
        std::vector<int> run;
        for (int gi = 0; gi < NGR; gi++) {
            const int gb = s->groups[gi]->B;
            if (pass == 0) {
                gfeed[gi].assign((size_t)std::max(nf_max, 1) * gb, 0);
                gnf[gi].assign(gb, 0);
                for (int b = 0; b < gb; b++) {
                    gnf[gi][b] = n_feed ? n_feed[r0[gi] + b] : n_feed_all;
                    for (int t = 0; t < gnf[gi][b] && t < nf_max; t++)
                        gfeed[gi][(size_t)t * gb + b] = feed[(size_t)t * B + r0[gi] + b];
                }
                run.push_back(gi);
            } else if (more[gi] > 0) {
                // feed each row its last id, then run greedily without a stop
                gfeed[gi].assign(gb, 0);
                gnf[gi].assign(gb, 1);
                for (int b = 0; b < gb; b++) gfeed[gi][b] = ids[(size_t)(done[gi] - 1) * B + r0[gi] + b];
                run.push_back(gi);
            }
        }
        if (run.empty()) continue;
        const int per = std::max(1, lead->grid_cap / (int)run.size());
        // every group is validated before any input is uploaded
        for (int gi : run) {
            const int rc = decode_launch(s->groups[gi], gfeed[gi].data(), 0, gnf[gi].data(), pass == 0 ? n_steps : more[gi],
                                         pass == 0 ? eos : -1, logits != nullptr, per, true);
            if (rc) return rc;
        }
        MultiArgs ma{};
        ma.n = (int)run.size();
        ma.per = per;
        for (int i = 0; i < ma.n; i++) {
            const int gi = run[i];
            const int rc = decode_launch(s->groups[gi], gfeed[gi].data(), 0, gnf[gi].data(), pass == 0 ? n_steps : more[gi],
                                         pass == 0 ? eos : -1, logits != nullptr, per, false, &ma.a[i]);
            if (rc) return rc;
        }
        const void *kern = decode_multi_for(m->ldD / LDALIGN);
        const size_t shmem = lds_bytes(MAXB, m->ldD, m->ldF);
        void *kargs[] = {&ma};
        HIP_TRY(hipEventRecord(lead->ev0, lead->stream));
        HIP_TRY(hipLaunchKernel(kern, dim3(per * ma.n), dim3(BLOCK), kargs, shmem, lead->stream));
        HIP_TRY(hipEventRecord(lead->ev1, lead->stream));
        HIP_TRY(hipEventSynchronize(lead->ev1));
        float pass_ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&pass_ms, lead->ev0, lead->ev1));
        ms += pass_ms;
        for (int gi : run) {
            dnn_hip_session *g = s->groups[gi];
            const int gb = g->B, steps = pass == 0 ? n_steps : more[gi];
            gids[gi].assign((size_t)steps * gb, 0);
            if (logits) glog[gi].assign((size_t)steps * gb * V, 0.f);
            int d = 0;
            const int rc = decode_finish(g, gids[gi].data(), logits ? glog[gi].data() : nullptr, &d, false);
            if (rc) return rc;
            g->last_ms = pass_ms;
            const int t0 = pass == 0 ? 0 : done[gi];
            for (int t = 0; t < d; t++)
                for (int b = 0; b < gb; b++) {
                    if (ids) ids[(size_t)(t0 + t) * B + r0[gi] + b] = gids[gi][(size_t)t * gb + b];
                    if (logits)
                        memcpy(logits + ((size_t)(t0 + t) * B + r0[gi] + b) * V, glog[gi].data() + ((size_t)t * gb + b) * V,
                               sizeof(float) * V);
                }
            if (pass == 0) done[gi] = d;
        }
    }
    s->last_ms = ms;
    if (steps_done) *steps_done = *std::max_element(done.begin(), done.end());
    return DNN_HIP_OK;
}

}  // namespace

int dnn_hip_decode(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed,
                   int n_steps, int eos, int *ids, float *logits, int *steps_done) {
    if (!s || !feed) return fail(DNN_HIP_EINVAL, "NULL argument");
    const int B = s->B;
    if (n_steps <= 0) return fail(DNN_HIP_EINVAL, "n_steps %d", n_steps);
    if (!s->groups.empty()) {
        if (!ids && eos >= 0) return fail(DNN_HIP_EINVAL, "a multi-group session needs ids when eos >= 0");
        for (int b = 0; b < B; b++)
            if ((n_feed ? n_feed[b] : n_feed_all) < 1)
                return fail(DNN_HIP_EINVAL, "row %d: n_feed %d < 1", b, n_feed ? n_feed[b] : n_feed_all);
        return decode_groups(s, feed, n_feed_all, n_feed, n_steps, eos, ids, logits, steps_done);
    }
    return decode_finish_launch(s, feed, n_feed_all, n_feed, n_steps, eos, ids, logits, steps_done);
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
