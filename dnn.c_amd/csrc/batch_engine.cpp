// batch_engine.cpp -- host side of the batched engine: buffers, the HIP graph
// of one decode step, multi-token prefill.
//
// Decode (dnn_hip_decode on a batched session) replays the captured step once
// per token: the per-step values (positions, the step counter, the next
// token's embedding row, the done flag) live in device memory and are advanced
// by the last workgroup of the lm_head kernel, so one graph serves every step.
// The graph holds no memset nodes: counters are reset by the kernels that use
// them.
//
// Prefill (dnn_hip_prefill) runs the new rows of every sequence through the
// layers at once -- the multi-token cached forward of the reference
// (transformer_block_forward_cached_ex, transformer.c:211-416, causal or
// prefix-LM), as decoder_lm_generate's prompt loop (gpt.c:306-344) and
// vision_lm_generate's prefix prefill (vlm.c:497-517) need it -- and returns the
// greedy token of each sequence's last new row.
#include <algorithm>
#include <array>
#include <cstring>
#include <vector>

#include "engine_plan.h"
#include "session.h"

using namespace dnnhip;

static_assert(PLAN_MAX_ROWS == MAX_ROWS, "the split-K plans cover every row count of a session");

namespace {

constexpr int CNT_ATT = MAX_ROWS * 64;   // (row, head) pairs of the decode attention
constexpr int CNT_TOTAL = CNT_GEMM + CNT_ATT + 1;

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return set_error(DNN_HIP_EDEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

inline int round_up(int v, int a) { return (v + a - 1) / a * a; }

// workgroups per (row, head) of the decode attention (attn_splits_for;
// DNN_HIP_ATT_SPLITS, read at session creation, overrides)
int attn_splits(const dnn_hip_session *s, int M, int H, int S_max) { return attn_splits_for(s->att_splits_req, M, H, S_max); }

// Split-K partial pairs of the engine: the largest need of any decode-shape
// GEMM launch at any row count (the prefill GEMMs never split K).
size_t engine_part_pairs(const dnn_hip_model *m) { return engine_part_need(m->D, m->F, m->V, m->ldD, m->ldF); }

void free_acts(BatchEngine *e) {
    float *bufs[] = {e->X, e->X1, e->ATT, e->Q, e->ACT};
    for (float *p : bufs)
        if (p) (void)hipFree(p);
    e->X = e->X1 = e->ATT = e->Q = e->ACT = nullptr;
    e->mcap = 0;
}

void drop_graph(BatchEngine *e) {
    if (e->gexec) (void)hipGraphExecDestroy(e->gexec);
    e->gexec = nullptr;
    e->gkey[0] = e->gkey[1] = e->gkey[2] = e->gkey[3] = nullptr;
}

// The session's engine with activation buffers of at least `rows` rows.
// The fragment-ordered weight copy the decode GEMMs read (built on the
// device from the arena at first use and after every weight upload).
int ensure_packed(dnn_hip_model *m, hipStream_t stream) {
    if (m->packed_valid) return DNN_HIP_OK;
    const size_t es = m->bf16 ? 2 : 4;
    auto elems = [](int N, int ld) { return (size_t)((N + 15) / 16) * 16 * (size_t)ld; };
    const int D = m->D, F = m->F, ldD = m->ldD, ldF = m->ldF;
    size_t o = 0;
    m->pk_embed = o;
    o += elems(m->V, ldD);
    m->pk_l.assign((size_t)m->L * 4, 0);
    for (int l = 0; l < m->L; l++) {
        size_t *p = &m->pk_l[(size_t)l * 4];
        p[0] = o; o += elems(3 * D, ldD);
        p[1] = o; o += elems(D, ldD);
        p[2] = o; o += elems(2 * F, ldD);
        p[3] = o; o += elems(D, ldF);
    }
    if (!m->packed || m->packed_bytes != o * es) {
        if (m->packed) (void)hipFree(m->packed);
        m->packed = nullptr;
        const hipError_t e = hipMalloc(&m->packed, o * es);
        if (e != hipSuccess) return set_error(DNN_HIP_ENOMEM, "hipMalloc(%zu) for the packed weights: %s", o * es, hipGetErrorString(e));
        m->packed_bytes = o * es;
    }
    const char *src = m->bf16 ? reinterpret_cast<const char *>(m->arena16) : m->arena;
    char *dst = static_cast<char *>(m->packed);
    const bool bf = m->bf16 != 0;
    HIP_TRY(launch_pack(src + m->off.embed / 4 * es, dst + m->pk_embed * es, m->V, ldD, bf, stream));
    for (int l = 0; l < m->L; l++) {
        const LayerOff &lo = m->h_layers[l];
        const size_t *p = &m->pk_l[(size_t)l * 4];
        HIP_TRY(launch_pack(src + (size_t)lo.wqkv * es, dst + p[0] * es, 3 * D, ldD, bf, stream));
        HIP_TRY(launch_pack(src + (size_t)lo.wo * es, dst + p[1] * es, D, ldD, bf, stream));
        HIP_TRY(launch_pack(src + (size_t)lo.wgu * es, dst + p[2] * es, 2 * F, ldD, bf, stream));
        HIP_TRY(launch_pack(src + (size_t)lo.wd * es, dst + p[3] * es, D, ldF, bf, stream));
    }
    HIP_TRY(hipStreamSynchronize(stream));
    m->packed_valid = true;
    return DNN_HIP_OK;
}

// The activation buffers' layout for the next launches: decode steps keep X,
// X1, ATT and ACT in fragment order, every other path row-major.  A change
// clears them, so the padding columns past d_model / d_ffn (summed into the
// folded rms_norm, met by zero weights) are zero in the new layout too.
int set_layout(dnn_hip_session *s, int layout) {
    BatchEngine *e = s->eng;
    if (e->layout == layout) return DNN_HIP_OK;
    const size_t ldD = s->m->ldD, ldF = s->m->ldF, mc = (size_t)e->mcap;
    HIP_TRY(hipMemsetAsync(e->X, 0, mc * ldD * 4, s->stream));
    HIP_TRY(hipMemsetAsync(e->X1, 0, mc * ldD * 4, s->stream));
    HIP_TRY(hipMemsetAsync(e->ATT, 0, mc * ldD * 4, s->stream));
    HIP_TRY(hipMemsetAsync(e->ACT, 0, mc * ldF * 4, s->stream));
    e->layout = layout;
    return DNN_HIP_OK;
}

// Clear the step state's step count and stop flag before a prefill, block or
// head launch: a decode call whose rows all stopped at eos leaves the flag set
// (its later graph replays skip their work), and the GEMMs and the finisher
// of these launches would skip theirs too.  A decode call clears both itself.
int clear_step(dnn_hip_session *s) {
    BatchEngine *e = s->eng;
    HIP_TRY(hipMemsetAsync(&e->st->t, 0, sizeof(int) * 2, s->stream));   // t, done
    return DNN_HIP_OK;
}

int engine_get(dnn_hip_session *s, int rows, int layout = 0) {
    dnn_hip_model *m = s->m;
    {
        const int rc = ensure_packed(m, s->stream);
        if (rc) return rc;
    }
    if (m->L * 5 + 1 >= 128) return set_error(DNN_HIP_EINVAL, "%d layers: the batched engine covers up to 25", m->L);
    if (m->H > 64) return set_error(DNN_HIP_EINVAL, "%d heads: the batched engine covers up to 64", m->H);
    if (m->V > 65535) return set_error(DNN_HIP_EINVAL, "vocab %d: the batched engine covers up to 65535", m->V);
    BatchEngine *e = s->eng;
    if (!e) {
        e = s->eng = new BatchEngine();
        const int ntn_head = (m->V + 15) / 16;
        e->part_pairs = engine_part_pairs(m);
        e->apart_pairs = (size_t)MAX_ROWS * m->H * 8 * (BK_DK + 2);
        e->amax_pairs = (size_t)MAX_ROWS * ntn_head + BK_MAXM;      // partials, then the finisher's stop records
        int rc = 0;
        rc = rc ? rc : dalloc(&e->part, e->part_pairs);
        rc = rc ? rc : dalloc(&e->apart, e->apart_pairs);
        rc = rc ? rc : dalloc(&e->amax, e->amax_pairs);
        rc = rc ? rc : dalloc(&e->cnt, CNT_TOTAL);
        rc = rc ? rc : dalloc(&e->st, 1);
        rc = rc ? rc : dalloc(&e->row_ident, MAX_ROWS);
        rc = rc ? rc : dalloc(&e->row_done, MAX_ROWS);
        rc = rc ? rc : dalloc(&e->steps_done, 1);
        rc = rc ? rc : dalloc(&e->next_ids, MAX_ROWS);
        rc = rc ? rc : dalloc(&e->pre_logits, (size_t)MAX_ROWS * m->V);
        if (rc) return rc;
        std::vector<int> ident(MAX_ROWS);
        for (int i = 0; i < MAX_ROWS; i++) ident[i] = i;
        StepState st0{1u, 0, 0, 0};   // tag 0 marks the zeroed partial buffers: never current
        HIP_TRY(hipMemset(e->part, 0, e->part_pairs * sizeof(uint2)));
        HIP_TRY(hipMemset(e->apart, 0, e->apart_pairs * sizeof(uint2)));
        HIP_TRY(hipMemset(e->amax, 0, e->amax_pairs * sizeof(uint2)));
        HIP_TRY(hipMemset(e->cnt, 0, CNT_TOTAL * sizeof(unsigned)));
        HIP_TRY(hipMemset(e->row_done, 0, MAX_ROWS * sizeof(int)));
        HIP_TRY(hipMemcpy(e->row_ident, ident.data(), MAX_ROWS * sizeof(int), hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(e->st, &st0, sizeof st0, hipMemcpyHostToDevice));
    }
    if (rows > e->mcap) {
        drop_graph(e);
        free_acts(e);
        const int mc = round_up(std::max(rows, BK_MAXM), BK_PBM);
        const size_t ldD = m->ldD, ldF = m->ldF;
        int rc = 0;
        rc = rc ? rc : dalloc(&e->X, mc * ldD);
        rc = rc ? rc : dalloc(&e->X1, mc * ldD);
        rc = rc ? rc : dalloc(&e->ATT, mc * ldD);
        rc = rc ? rc : dalloc(&e->Q, mc * (size_t)m->D);
        rc = rc ? rc : dalloc(&e->ACT, mc * ldF);
        if (rc) { free_acts(e); return rc; }
        // padding columns (past d_model / d_ffn) stay zero: they meet the
        // weights' zero padding in the k-loops
        HIP_TRY(hipMemset(e->X, 0, mc * ldD * 4));
        HIP_TRY(hipMemset(e->X1, 0, mc * ldD * 4));
        HIP_TRY(hipMemset(e->ATT, 0, mc * ldD * 4));
        HIP_TRY(hipMemset(e->Q, 0, mc * (size_t)m->D * 4));
        HIP_TRY(hipMemset(e->ACT, 0, mc * ldF * 4));
        e->mcap = mc;
        e->layout = 0;
    }
    return set_layout(s, layout);
}

// Attention tiles (batch row, first new row) of a prefill, heaviest first: by
// the keys the tile's last row sees, as prefill_attn_kernel counts them, ties
// in building order.  The kernel's workgroups are dispatched tile-major, so
// the longest start first and the launch ends on the shortest.
std::vector<int> prefill_tiles(int B, const int *nn, const int *p0, int mode, int prefix_len) {
    std::vector<std::array<int, 3>> t;
    for (int b = 0; b < B; b++)
        for (int t0 = 0; t0 < nn[b]; t0 += 64) {
            int kv_end = p0[b] + t0 + std::min(64, nn[b] - t0);
            if (mode == 1 && kv_end < prefix_len) kv_end = prefix_len;
            t.push_back({std::min(kv_end, p0[b] + nn[b]), b, t0});
        }
    std::stable_sort(t.begin(), t.end(), [](const std::array<int, 3> &x, const std::array<int, 3> &y) { return x[0] > y[0]; });
    std::vector<int> out;
    for (const auto &x : t) { out.push_back(x[1]); out.push_back(x[2]); }
    return out;
}

struct Wts {
    const dnn_hip_model *m;
    const float *f(uint32_t off) const { return reinterpret_cast<const float *>(m->arena) + off; }
};

GemmArgs gemm_base(dnn_hip_session *s, size_t pk, int ldw, int N, int K) {
    GemmArgs g{};
    const size_t es = s->m->bf16 ? 2 : 4;
    g.Wp = static_cast<const char *>(s->m->packed) + pk * es;
    g.wp_bytes = (size_t)((N + 15) / 16) * 16 * (size_t)ldw * es;
    g.ldw = ldw;
    g.N = N;
    g.K = K;
    g.ks = 1;
    g.st = s->eng->st;
    g.mpad = s->eng->mcap;
    g.D = s->m->D;
    g.part_cap = s->eng->part_pairs;
    g.cnt_cap = CNT_GEMM;
    return g;
}

// The launches of one layer: QKV, attention, out_proj, gate/up, down.  decode:
// M = the session's rows, the attention of each row over its cache; prefill:
// M = the packed new rows (pi: host-side prefill plan in device memory).
struct PrefillPlan {
    int M;
    const int *row_b, *row_p, *pid, *row0, *n_new, *p0, *arow, *tiles;
    int n_tiles, mode, prefix_len;
    int pk;             // activations in fragment order (engine_prefill), else row-major
};

int enqueue_layer(dnn_hip_session *s, int l, const PrefillPlan *pp) {
    dnn_hip_model *m = s->m;
    BatchEngine *e = s->eng;
    const Wts W{m};
    const LayerOff &lo = m->h_layers[l];
    const int D = m->D, ldD = m->ldD, ldF = m->ldF;
    const bool pre = pp != nullptr;
    const int pk = !pre || pp->pk;          // activations in fragment order
    const int M = pre ? pp->M : s->B;
    const bool bf = m->bf16 != 0;
    const MtPlan mp = mt_plan(M, true);
    // GEMM shape: the prefill tiles (128 rows) only for more rows than one
    // decode-shape launch takes; fewer prefill rows run the decode-shape
    // GEMMs (16-row tiles, K split over wavefronts and workgroups) like a
    // decode step of M rows (a 32-token prompt: 3.0 -> 0.5 ms)
    const bool ps = pre && M > BK_MAXM;

    GemmArgs g = gemm_base(s, m->pk_l[(size_t)l * 4 + 0], ldD, 3 * D, ldD);
    g.A = e->X; g.lda = ldD; g.M = M;
    if (!ps) g.mt_max = mp.qkv;
    g.ks = ps ? 1 : pick_ks((3 * D + 15) / 16, ldD, M, true, g.mt_max);
    g.part = e->part; g.cnt = e->cnt;
    g.bias = W.f(lo.bqkv);
    g.gamma = W.f(lo.g_attn); g.eps = lo.eps_attn; g.dnorm = D;
    g.q = e->Q; g.kc = s->kc; g.vc = s->vc;
    g.row_b = pre ? pp->row_b : e->row_ident;
    g.row_p = pre ? pp->row_p : s->pos;
    g.H = m->H; g.kv_s = s->kv_s; g.B = s->B; g.layer = l;
    g.rope = m->rope; g.rope_rows = m->rope_rows;
    g.kslot = 5 * l;
    g.pk = pk;
    HIP_TRY(launch_gemm(EPI_QKV, true, bf, ps, g, s->stream));

    if (pre) {
        PrefillAttnArgs a{};
        a.q = e->Q; a.att = e->ATT; a.kc = s->kc; a.vc = s->vc;
        a.row0 = pp->row0; a.n_new = pp->n_new; a.p0 = pp->p0; a.tiles = pp->tiles;
        a.n_tiles = pp->n_tiles; a.H = m->H; a.kv_s = s->kv_s; a.layer = l; a.D = D; a.B = s->B; a.ldatt = ldD;
        a.mode = pp->mode; a.prefix_len = pp->prefix_len; a.st = e->st; a.pk = pk;
        HIP_TRY(launch_prefill_attn(a, s->stream));
    } else {
        AttnArgs a{};
        a.q = e->Q; a.att = e->ATT; a.kc = s->kc; a.vc = s->vc; a.pos = s->pos;
        a.M = M; a.H = m->H; a.kv_s = s->kv_s; a.layer = l; a.D = D; a.B = s->B; a.ldatt = ldD;
        a.nsplit = e->att_ns;
        a.part = e->apart; a.cnt = e->cnt + CNT_GEMM; a.st = e->st; a.kslot = 5 * l + 1;
        a.pk = 1;                               // decode steps: ATT in fragment order
        a.spec = e->att_spec;
        HIP_TRY(launch_attn(a, s->stream));
    }

    g = gemm_base(s, m->pk_l[(size_t)l * 4 + 1], ldD, D, ldD);
    g.A = e->ATT; g.lda = ldD; g.M = M;
    g.bias = W.f(lo.bo);
    g.out = e->X1; g.ldo = ldD; g.res = e->X; g.ldr = ldD;
    if (!ps) g.mt_max = mp.out;
    g.ks = ps ? 1 : pick_ks((D + 15) / 16, ldD, M, false, g.mt_max);
    g.part = e->part; g.cnt = e->cnt; g.kslot = 5 * l + 2;
    g.pk = pk;
    HIP_TRY(launch_gemm(EPI_RES, false, bf, ps, g, s->stream));

    g = gemm_base(s, m->pk_l[(size_t)l * 4 + 2], ldD, 2 * m->F, ldD);
    g.A = e->X1; g.lda = ldD; g.M = M;
    g.bias = W.f(lo.bg); g.bias2 = W.f(lo.bu);
    g.gamma = W.f(lo.g_ffn); g.eps = lo.eps_ffn; g.dnorm = D;
    g.out = e->ACT; g.ldo = ldF;
    if (!ps) g.mt_max = mp.gu;
    g.ks = ps ? 1 : pick_ks((2 * m->F + 15) / 16, ldD, M, true, g.mt_max);
    g.part = e->part; g.cnt = e->cnt;
    g.kslot = 5 * l + 3;
    g.pk = pk;
    HIP_TRY(launch_gemm(EPI_SWIGLU, true, bf, ps, g, s->stream));

    g = gemm_base(s, m->pk_l[(size_t)l * 4 + 3], ldF, D, ldF);
    g.A = e->ACT; g.lda = ldF; g.M = M;
    g.bias = W.f(lo.bd);
    g.out = e->X; g.ldo = ldD; g.res = e->X1; g.ldr = ldD;
    if (!ps) g.mt_max = mp.down;
    g.ks = ps ? 1 : pick_ks((D + 15) / 16, ldF, M, false, g.mt_max);
    g.part = e->part; g.cnt = e->cnt; g.kslot = 5 * l + 4;
    g.pk = pk;
    HIP_TRY(launch_gemm(EPI_RES, false, bf, ps, g, s->stream));
    return DNN_HIP_OK;
}

// final rms_norm -> tied lm_head -> argmax (+ the next step's feed in decode)
int enqueue_head(dnn_hip_session *s, const PrefillPlan *pp, float *logits, int *ids, int eos, int rows = 0,
                 bool norm = true) {
    dnn_hip_model *m = s->m;
    BatchEngine *e = s->eng;
    const Wts W{m};
    const uint32_t embed = (uint32_t)(m->off.embed / 4), lm_bias = (uint32_t)(m->off.lm_bias / 4),
                   g_final = (uint32_t)(m->off.g_final / 4);
    GemmArgs g = gemm_base(s, m->pk_embed, m->ldD, m->V, m->ldD);
    g.A = e->X; g.lda = m->ldD; g.M = rows > 0 ? rows : s->B;
    g.arow = pp ? pp->arow : nullptr;
    g.bias = W.f(lm_bias);
    g.gamma = norm ? W.f(g_final) : nullptr; g.eps = m->eps_final; g.dnorm = m->D;
    g.amax = e->amax; g.head_cnt = e->cnt + CNT_GEMM + CNT_ATT;
    g.fin = e->amax + (size_t)MAX_ROWS * ((m->V + 15) / 16);
    g.logits = logits; g.ids = ids;
    g.feed = s->feed; g.n_feed = s->n_feed; g.pos = s->pos;
    g.x_next = e->X; g.ldx = m->ldD; g.embed = W.f(embed);
    g.steps_done = e->steps_done; g.eos = eos; g.row_done = e->row_done;
    g.prefill = pp != nullptr;
    g.pk = pp == nullptr || pp->pk;          // decode steps and prefill: X in fragment order
    g.kslot = 5 * m->L;
    g.mt_max = mt_plan(g.M, pp == nullptr).head;
    g.ks = pick_ks((m->V + 15) / 16, m->ldD, g.M, true, g.mt_max);
    g.amax_tiles = (m->V + 15) / 16;
    g.part = e->part; g.cnt = e->cnt;
    HIP_TRY(launch_gemm(EPI_HEAD, norm, m->bf16 != 0, false, g, s->stream));
    HIP_TRY(launch_head_finish(g, s->stream));
    return DNN_HIP_OK;
}

}  // namespace

namespace dnnhip {

void engine_destroy(BatchEngine *e) {
    if (!e) return;
    drop_graph(e);
    free_acts(e);
    void *bufs[] = {e->part, e->apart, e->amax, e->cnt, e->st, e->row_ident, e->row_done,
                    e->steps_done, e->pre_i, e->next_ids, e->pre_logits};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    delete e;
}

int engine_decode(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps, int eos,
                  int *ids, float *logits, int *steps_done) {
    dnn_hip_model *m = s->m;
    const int B = s->B;
    std::vector<int> nf;
    int nf_max = 0;
    int rc = check_decode(s, feed, n_feed_all, n_feed, n_steps, nf, &nf_max);
    if (rc) return rc;
    HIP_TRY(hipSetDevice(m->device));
    rc = engine_get(s, round_up(B, 16), 1);
    if (!rc) rc = grow(&s->feed, &s->feed_cap, (size_t)nf_max * B);
    if (!rc) rc = grow(&s->ids, &s->ids_cap, (size_t)n_steps * B);
    if (!rc && logits) rc = grow(&s->logits, &s->logits_cap, (size_t)n_steps * B * m->V);
    if (rc) return rc;
    BatchEngine *e = s->eng;
    {
        const size_t feed_bytes = sizeof(int) * (size_t)nf_max * B, nf_bytes = sizeof(int) * B;
        rc = stage_begin(s, stage_size(feed_bytes) + stage_size(nf_bytes));
        if (!rc) rc = stage_copy(s, s->feed, feed, feed_bytes);
        if (!rc) rc = stage_copy(s, s->n_feed, nf.data(), nf_bytes);
        if (rc) return rc;
    }

    // the decode attention's key splits and speculative first-chunk loads
    {
        int s_max = 0;
        for (int b = 0; b < B; b++) s_max = std::max(s_max, s->h_pos[b] + n_steps);
        const int ns = attn_splits(s, B, m->H, s_max);
        e->att_ns = ns;
        s->att_splits = ns;
        e->att_spec = attn_spec(attn_waves(B, m->H), ns, B, n_steps, s->h_pos.data());
    }
    // the step graph, captured again when a buffer it names or a launch
    // parameter changed.  DNN_HIP_ENGINE_GRAPH=0 launches the step's kernels
    // directly instead (the same kernels and arguments; every per-step value
    // lives in device memory either way) -- for tools that trace kernel
    // dispatches one by one.
    const char *graph_env = getenv("DNN_HIP_ENGINE_GRAPH");
    const bool use_graph = !(graph_env && graph_env[0] == '0');
    float *lg = logits ? s->logits : nullptr;
    const void *key[4] = {s->feed, s->ids, lg, e->X};
    if (use_graph && (!e->gexec || e->geos != eos || e->gspec != e->att_spec || e->gns != e->att_ns ||
                      memcmp(key, e->gkey, sizeof key) != 0)) {
        drop_graph(e);
        HIP_TRY(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
        int erc = 0;
        for (int l = 0; l < m->L && !erc; l++) erc = enqueue_layer(s, l, nullptr);
        if (!erc) erc = enqueue_head(s, nullptr, lg, s->ids, eos);
        hipGraph_t graph = nullptr;
        const hipError_t ce = hipStreamEndCapture(s->stream, &graph);
        if (erc) { if (graph) (void)hipGraphDestroy(graph); return erc; }
        if (ce != hipSuccess) return set_error(DNN_HIP_EDEVICE, "step graph capture: %s", hipGetErrorString(ce));
        const hipError_t ie = hipGraphInstantiate(&e->gexec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (ie != hipSuccess) { e->gexec = nullptr; return set_error(DNN_HIP_EDEVICE, "step graph: %s", hipGetErrorString(ie)); }
        memcpy(e->gkey, key, sizeof key);
        e->geos = eos;
        e->gspec = e->att_spec;
        e->gns = e->att_ns;
    }
    // the first step's embedding rows; resets the step counter, done flags
    EmbedArgs ea{};
    ea.embed = reinterpret_cast<const float *>(m->arena) + m->off.embed / 4;
    ea.ids = s->feed; ea.out = e->X; ea.M = B; ea.ld = m->ldD; ea.D = m->D; ea.st = e->st; ea.row_done = e->row_done;
    ea.pk = 1;                               // decode steps keep X in fragment order
    HIP_TRY(launch_embed(ea, s->stream));
    HIP_TRY(hipEventRecord(s->ev0, s->stream));
    for (int t = 0; t < n_steps; t++) {
        if (use_graph) {
            HIP_TRY(hipGraphLaunch(e->gexec, s->stream));
            continue;
        }
        for (int l = 0; l < m->L; l++) {
            rc = enqueue_layer(s, l, nullptr);
            if (rc) return rc;
        }
        rc = enqueue_head(s, nullptr, lg, s->ids, eos);
        if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(s->ev1, s->stream));
    HIP_TRY(hipEventSynchronize(s->ev1));
    HIP_TRY(hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1));
    s->kernel_used = 6;
    int done = 0;
    HIP_TRY(hipMemcpy(&done, e->steps_done, sizeof(int), hipMemcpyDeviceToHost));
    if (done < 1 || done > n_steps) return set_error(DNN_HIP_EDEVICE, "batched decode: %d of %d steps reported", done, n_steps);
    if (ids) HIP_TRY(hipMemcpy(ids, s->ids, sizeof(int) * (size_t)done * B, hipMemcpyDeviceToHost));
    if (logits) HIP_TRY(hipMemcpy(logits, s->logits, sizeof(float) * (size_t)done * B * m->V, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(s->h_pos.data(), s->pos, sizeof(int) * B, hipMemcpyDeviceToHost));
    if (steps_done) *steps_done = done;
    return DNN_HIP_OK;
}

int engine_prefill(dnn_hip_session *s, const float *embeds, int n_embed, const int *ids, int n_ids_max,
                   const int *n_ids, int mode, int prefix_len, int *next_ids, float *logits) {
    dnn_hip_model *m = s->m;
    const int B = s->B, D = m->D;
    if (n_embed < 0 || n_ids_max < 0) return set_error(DNN_HIP_EINVAL, "n_embed %d / n_ids_max %d", n_embed, n_ids_max);
    if (n_embed > 0 && !embeds) return set_error(DNN_HIP_EINVAL, "embeds is NULL");
    if (mode != 0 && mode != 1) return set_error(DNN_HIP_EINVAL, "mode %d: 0 (causal) or 1 (prefix-LM)", mode);
    std::vector<int> nn(B), row0(B), p0(B), arow(B);
    int M = 0;
    for (int b = 0; b < B; b++) {
        const int ni = n_ids ? n_ids[b] : n_ids_max;
        if (ni < 0 || ni > n_ids_max) return set_error(DNN_HIP_EINVAL, "row %d: %d ids of at most %d", b, ni, n_ids_max);
        if (ni > 0 && !ids) return set_error(DNN_HIP_EINVAL, "ids is NULL");
        for (int t = 0; t < ni; t++) {
            const int id = ids[(size_t)b * n_ids_max + t];
            if (id < 0 || id >= m->V) return set_error(DNN_HIP_ERANGE, "token id %d at row %d position %d outside [0,%d)", id, b, t, m->V);
        }
        nn[b] = n_embed + ni;
        if (nn[b] < 1) return set_error(DNN_HIP_EINVAL, "row %d: no new rows", b);
        p0[b] = s->h_pos[b];
        if (mode == 1 && p0[b] != 0) return set_error(DNN_HIP_EINVAL, "prefix-LM prefill needs an empty cache (row %d holds %d)", b, p0[b]);
        if (p0[b] + nn[b] > s->max_seq)
            return set_error(DNN_HIP_ERANGE, "row %d: %d cached + %d new exceeds max_seq %d", b, p0[b], nn[b], s->max_seq);
        if (m->rope && p0[b] + nn[b] > m->rope_rows)
            return set_error(DNN_HIP_ERANGE, "row %d: position %d beyond the RoPE table (%d rows)", b, p0[b] + nn[b] - 1, m->rope_rows);
        row0[b] = M;
        arow[b] = M + nn[b] - 1;
        M += nn[b];
    }
    HIP_TRY(hipSetDevice(m->device));
    int rc = engine_get(s, M, 1);            // activations in fragment order, as decode keeps them
    if (!rc) rc = clear_step(s);
    if (rc) return rc;
    BatchEngine *e = s->eng;
    // the plan: row_b, row_p, pid [M]; row0, n_new, p0, arow [B]; tiles [T][2]
    const std::vector<int> tiles = prefill_tiles(B, nn.data(), p0.data(), mode, prefix_len);
    const int T = (int)tiles.size() / 2;
    std::vector<int> plan((size_t)3 * M + 4 * B + tiles.size());
    int *row_b = plan.data(), *row_p = row_b + M, *pid = row_p + M, *hrow0 = pid + M, *hnn = hrow0 + B,
        *hp0 = hnn + B, *harow = hp0 + B, *htiles = harow + B;
    for (int b = 0; b < B; b++) {
        const int ni = nn[b] - n_embed;
        for (int t = 0; t < nn[b]; t++) {
            const int r = row0[b] + t;
            row_b[r] = b;
            row_p[r] = p0[b] + t;
            pid[r] = t < n_embed ? -1 : ids[(size_t)b * n_ids_max + (t - n_embed)];
        }
        (void)ni;
        hrow0[b] = row0[b]; hnn[b] = nn[b]; hp0[b] = p0[b]; harow[b] = arow[b];
    }
    std::copy(tiles.begin(), tiles.end(), htiles);
    rc = grow(&e->pre_i, &e->pre_cap, plan.size());
    if (rc) return rc;
    const size_t emb_row = (size_t)D * 4 * n_embed;
    rc = stage_begin(s, stage_size(plan.size() * sizeof(int)) + (size_t)B * stage_size(emb_row));
    if (!rc) rc = stage_copy(s, e->pre_i, plan.data(), plan.size() * sizeof(int));
    if (rc) return rc;
    int *d = e->pre_i;
    PrefillPlan pp{M, d, d + M, d + 2 * M, d + 3 * M, d + 3 * M + B, d + 3 * M + 2 * B, d + 3 * M + 3 * B,
                   d + 3 * M + 4 * B, T, mode, prefix_len, 1};
    // embedding inputs (e.g. image patches) staged row-major in the attention
    // buffer (free until the first layer's attention), then every row into X
    // in fragment order: those copied, token rows gathered
    if (n_embed > 0)
        for (int b = 0; b < B && !rc; b++)
            rc = stage_copy2d(s, e->ATT + (size_t)row0[b] * m->ldD, (size_t)m->ldD * 4, embeds + (size_t)b * n_embed * D,
                              (size_t)D * 4, (size_t)D * 4, n_embed);
    if (rc) return rc;
    EmbedArgs ea{};
    ea.embed = reinterpret_cast<const float *>(m->arena) + m->off.embed / 4;
    ea.ids = pp.pid; ea.out = e->X; ea.M = M; ea.ld = m->ldD; ea.D = D;
    ea.src = n_embed > 0 ? e->ATT : nullptr;
    ea.pk = 1;
    HIP_TRY(launch_embed(ea, s->stream));
    HIP_TRY(hipEventRecord(s->ev0, s->stream));
    for (int l = 0; l < m->L; l++) {
        rc = enqueue_layer(s, l, &pp);
        if (rc) return rc;
    }
    rc = enqueue_head(s, &pp, logits ? e->pre_logits : nullptr, e->next_ids, -1);
    if (rc) return rc;
    HIP_TRY(hipEventRecord(s->ev1, s->stream));
    HIP_TRY(hipEventSynchronize(s->ev1));
    HIP_TRY(hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1));
    HIP_TRY(hipMemcpy(next_ids, e->next_ids, sizeof(int) * B, hipMemcpyDeviceToHost));
    if (logits) HIP_TRY(hipMemcpy(logits, e->pre_logits, sizeof(float) * (size_t)B * m->V, hipMemcpyDeviceToHost));
    for (int b = 0; b < B; b++) s->h_pos[b] = p0[b] + nn[b];
    HIP_TRY(hipMemcpy(s->pos, s->h_pos.data(), sizeof(int) * B, hipMemcpyHostToDevice));
    return DNN_HIP_OK;
}


// One block over n_new rows of every batch row at positions pos0.. (the
// reference's per-layer cached forward: the caller's cache length is pos0).
int engine_block(dnn_hip_session *s, int layer, const float *x, int n_new, int pos0, int mode, int prefix_len,
                 float *y) {
    dnn_hip_model *m = s->m;
    const int B = s->B, D = m->D, M = B * n_new;
    if (layer < 0 || layer >= m->L) return set_error(DNN_HIP_EINVAL, "layer %d of %d", layer, m->L);
    if (!x || !y || n_new < 1 || pos0 < 0) return set_error(DNN_HIP_EINVAL, "bad block input (n_new %d, pos0 %d)", n_new, pos0);
    if (mode != 0 && mode != 1) return set_error(DNN_HIP_EINVAL, "mode %d: 0 (causal) or 1 (prefix-LM)", mode);
    if (mode == 1 && pos0 != 0) return set_error(DNN_HIP_EINVAL, "prefix-LM needs an empty cache (position %d)", pos0);
    if (pos0 + n_new > s->max_seq)
        return set_error(DNN_HIP_ERANGE, "%d cached + %d new exceeds max_seq %d", pos0, n_new, s->max_seq);
    if (m->rope && pos0 + n_new > m->rope_rows)
        return set_error(DNN_HIP_ERANGE, "position %d beyond the RoPE table (%d rows)", pos0 + n_new - 1, m->rope_rows);
    HIP_TRY(hipSetDevice(m->device));
    int rc = engine_get(s, M);
    if (!rc) rc = clear_step(s);
    if (rc) return rc;
    BatchEngine *e = s->eng;
    const std::vector<int> bn(B, n_new), bp(B, pos0);
    const std::vector<int> tiles = prefill_tiles(B, bn.data(), bp.data(), mode, prefix_len);
    const int T = (int)tiles.size() / 2;
    std::vector<int> plan((size_t)3 * M + 4 * B + tiles.size());
    int *row_b = plan.data(), *row_p = row_b + M, *pid = row_p + M, *hrow0 = pid + M, *hnn = hrow0 + B,
        *hp0 = hnn + B, *harow = hp0 + B, *htiles = harow + B;
    for (int b = 0; b < B; b++) {
        for (int t = 0; t < n_new; t++) {
            row_b[b * n_new + t] = b;
            row_p[b * n_new + t] = pos0 + t;
            pid[b * n_new + t] = -1;
        }
        hrow0[b] = b * n_new; hnn[b] = n_new; hp0[b] = pos0; harow[b] = b * n_new + n_new - 1;
    }
    std::copy(tiles.begin(), tiles.end(), htiles);
    rc = grow(&e->pre_i, &e->pre_cap, plan.size());
    if (rc) return rc;
    rc = stage_begin(s, stage_size(plan.size() * sizeof(int)) + stage_size((size_t)D * 4 * M));
    if (!rc) rc = stage_copy(s, e->pre_i, plan.data(), plan.size() * sizeof(int));
    if (!rc) rc = stage_copy2d(s, e->X, (size_t)m->ldD * 4, x, (size_t)D * 4, (size_t)D * 4, M);
    if (rc) return rc;
    int *d = e->pre_i;
    PrefillPlan pp{M, d, d + M, d + 2 * M, d + 3 * M, d + 3 * M + B, d + 3 * M + 2 * B, d + 3 * M + 3 * B,
                   d + 3 * M + 4 * B, T, mode, prefix_len};
    HIP_TRY(hipEventRecord(s->ev0, s->stream));
    rc = enqueue_layer(s, layer, &pp);
    if (rc) return rc;
    HIP_TRY(hipEventRecord(s->ev1, s->stream));
    HIP_TRY(hipMemcpy2DAsync(y, (size_t)D * 4, e->X, (size_t)m->ldD * 4, (size_t)D * 4, M, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    HIP_TRY(hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1));
    return DNN_HIP_OK;
}

// logits [n][V] of n rows (optionally through the final rms_norm first), in
// chunks of up to 64 rows of the decode-shape lm_head GEMM.
int engine_head(dnn_hip_session *s, const float *x, int n, int norm, float *logits) {
    dnn_hip_model *m = s->m;
    const int D = m->D;
    if (!x || !logits || n < 1) return set_error(DNN_HIP_EINVAL, "bad head input (%d rows)", n);
    HIP_TRY(hipSetDevice(m->device));
    int rc = engine_get(s, n);
    if (!rc) rc = clear_step(s);
    if (rc) return rc;
    BatchEngine *e = s->eng;
    std::vector<int> rows(n);
    for (int i = 0; i < n; i++) rows[i] = i;
    rc = grow(&e->pre_i, &e->pre_cap, (size_t)n);
    if (rc) return rc;
    rc = stage_begin(s, stage_size((size_t)n * sizeof(int)) + stage_size((size_t)D * 4 * n));
    if (!rc) rc = stage_copy(s, e->pre_i, rows.data(), (size_t)n * sizeof(int));
    if (!rc) rc = stage_copy2d(s, e->X, (size_t)m->ldD * 4, x, (size_t)D * 4, (size_t)D * 4, n);
    if (rc) return rc;
    for (int r0 = 0; r0 < n; r0 += BK_MAXM) {
        const int cnt = std::min(BK_MAXM, n - r0);
        PrefillPlan pp{};
        pp.arow = e->pre_i + r0;
        rc = enqueue_head(s, &pp, e->pre_logits, e->next_ids, -1, cnt, norm != 0);
        if (rc) return rc;
        HIP_TRY(hipMemcpyAsync(logits + (size_t)r0 * m->V, e->pre_logits, sizeof(float) * (size_t)cnt * m->V,
                               hipMemcpyDeviceToHost, s->stream));
    }
    HIP_TRY(hipStreamSynchronize(s->stream));
    return DNN_HIP_OK;
}

// Embedding rows of n token ids (embedding.c:79-84) into out [n][d_model].
int engine_embed(dnn_hip_session *s, const int *ids, int n, float *out) {
    dnn_hip_model *m = s->m;
    if (!ids || !out || n < 1) return set_error(DNN_HIP_EINVAL, "bad embedding input (%d ids)", n);
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->V) return set_error(DNN_HIP_ERANGE, "token id %d outside [0,%d)", ids[i], m->V);
    HIP_TRY(hipSetDevice(m->device));
    int rc = engine_get(s, n);
    if (rc) return rc;
    BatchEngine *e = s->eng;
    rc = grow(&e->pre_i, &e->pre_cap, (size_t)n);
    if (rc) return rc;
    rc = stage_begin(s, stage_size((size_t)n * sizeof(int)));
    if (!rc) rc = stage_copy(s, e->pre_i, ids, (size_t)n * sizeof(int));
    if (rc) return rc;
    EmbedArgs ea{};
    ea.embed = reinterpret_cast<const float *>(m->arena) + m->off.embed / 4;
    ea.ids = e->pre_i; ea.out = e->X; ea.M = n; ea.ld = m->ldD; ea.D = m->D;
    HIP_TRY(launch_embed(ea, s->stream));
    HIP_TRY(hipMemcpy2DAsync(out, (size_t)m->D * 4, e->X, (size_t)m->ldD * 4, (size_t)m->D * 4, n, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return DNN_HIP_OK;
}

// rms_norm of n rows of d values with a caller's gamma (rms_norm_forward,
// nn.c:169-173): x, gamma, y in host memory.
int engine_rms_norm(dnn_hip_session *s, const float *x, const float *gamma, int n, int d, float eps, float *y) {
    dnn_hip_model *m = s->m;
    if (!x || !gamma || !y || n < 1 || d < 1 || d > m->ldD) return set_error(DNN_HIP_EINVAL, "bad rms_norm input (%d x %d)", n, d);
    HIP_TRY(hipSetDevice(m->device));
    int rc = engine_get(s, n);
    if (rc) return rc;
    BatchEngine *e = s->eng;
    float *g = e->X1;                                  // gamma in row 0 of X1, rows of x in X, y into ATT
    rc = stage_begin(s, stage_size(sizeof(float) * d) + stage_size((size_t)d * 4 * n));
    if (!rc) rc = stage_copy(s, g, gamma, sizeof(float) * d);
    if (!rc) rc = stage_copy2d(s, e->X, (size_t)m->ldD * 4, x, (size_t)d * 4, (size_t)d * 4, n);
    if (rc) return rc;
    HIP_TRY(launch_rms_rows(e->X, g, e->ATT, n, d, m->ldD, eps, s->stream));
    HIP_TRY(hipMemcpy2DAsync(y, (size_t)d * 4, e->ATT, (size_t)m->ldD * 4, (size_t)d * 4, n, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return DNN_HIP_OK;
}

}  // namespace dnnhip
