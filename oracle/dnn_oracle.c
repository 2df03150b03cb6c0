/*
 * dnn_oracle.c -- CPU restatement of masc-it/dnn.c's GPT decode path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT: the checker for the HIP path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Each function names the reference file:line whose arithmetic it restates.  The
 * float operation order and rounding are the reference's; only loop nests that
 * leave every output's own operation sequence unchanged were reordered (e.g. the
 * GEMV walks W row by row, but every y[j] is still one sequential k-chain of
 * rounded multiplies and adds, as in ops_matrix.c:1143-1151).
 *
 * Pinning (tests/test_oracle_golden.py): RNG, init, RoPE tables, every single op,
 * the cached block, prefix-LM prefill, no-cache forward and end-to-end greedy
 * generation are compared bit-for-bit with fixtures written by the reference
 * itself (oracle/_ref, built from /root/reference/src by oracle/Makefile).
 * libm-dependent bits (expf, logf, cosf, sinf, powf) are pinned only for the
 * glibc the fixtures were made with; the tests re-check them on every host.
 */
#include "dnn_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <assert.h>

/* ------------------------------------------------------------------ RNG */

static uint64_t xs128p(orc_rng *r) {               /* rng.c:6-13 */
    uint64_t s1 = r->s[0];
    uint64_t s0 = r->s[1];
    r->s[0] = s0;
    s1 ^= s1 << 23;
    r->s[1] = s1 ^ s0 ^ (s1 >> 18) ^ (s0 >> 5);
    return r->s[1] + s0;
}

static uint64_t splitmix_round(uint64_t x) {         /* rng.c:17-29 */
    uint64_t z = x + 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

void orc_rng_seed(orc_rng *r, uint64_t seed) {
    r->s[0] = splitmix_round(seed);
    r->s[1] = splitmix_round(r->s[0]);
}

float orc_rng_uniform(orc_rng *r) {                  /* rng.c:33-36 */
    return (float)(xs128p(r) >> 11) * 0x1.0p-53f;
}

float orc_rng_normal(orc_rng *r) {                   /* rng.c:40-47 */
    float u1, u2;
    do { u1 = orc_rng_uniform(r); } while (u1 == 0.0f);
    u2 = orc_rng_uniform(r);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

int orc_rng_uniform_int(orc_rng *r, int n) {         /* rng.c:51-66 */
    if (n <= 1) return 0;
    uint32_t limit = (uint32_t)n, mask = limit;
    mask |= mask >> 1; mask |= mask >> 2; mask |= mask >> 4;
    mask |= mask >> 8; mask |= mask >> 16;
    uint32_t v;
    do { v = (uint32_t)(xs128p(r) >> 32) & mask; } while (v >= limit);
    return (int)v;
}

/* The reference's default stream: _Thread_local, seeded {1,2} (rng.c:70-78). */
static _Thread_local orc_rng g_rng = { { 1, 2 } };

/* --------------------------------------------------------------- model */

#define NPL 12   /* parameter tensors per block, module order (transformer.c:116-147) */

orc_model *orc_model_create(const orc_cfg *cfg) {
    assert(cfg->D == cfg->H * cfg->dk);
    orc_model *m = calloc(1, sizeof(*m));
    m->cfg = *cfg;
    long long V = cfg->V, D = cfg->D, F = cfg->F, L = cfg->L;
    long long per_layer = D * 3 * D + 3 * D + D * D + D + 2 * D + 2 * (D * F + F) + F * D + D;
    m->n_floats = V * D + L * per_layer + D + V;
    m->arena = calloc((size_t)m->n_floats, sizeof(float));
    m->layers = calloc((size_t)L, sizeof(orc_layer));
    float *p = m->arena;
#define TAKE(n) (p += (n), p - (n))
    m->embed = TAKE(V * D);
    for (int l = 0; l < L; l++) {
        orc_layer *ly = &m->layers[l];
        ly->wqkv = TAKE(D * 3 * D); ly->bqkv = TAKE(3 * D);
        ly->wo = TAKE(D * D);       ly->bo = TAKE(D);
        ly->g_attn = TAKE(D);       ly->g_ffn = TAKE(D);
        ly->wg = TAKE(D * F);       ly->bg = TAKE(F);
        ly->wu = TAKE(D * F);       ly->bu = TAKE(F);
        ly->wd = TAKE(F * D);       ly->bd = TAKE(D);
    }
    m->g_final = TAKE(D);
    m->lm_bias = TAKE(V);
#undef TAKE
    assert(p == m->arena + m->n_floats);
    for (int l = 0; l < L; l++)
        for (int i = 0; i < D; i++) m->layers[l].g_attn[i] = m->layers[l].g_ffn[i] = 1.0f;
    for (int i = 0; i < D; i++) m->g_final[i] = 1.0f;
    if (cfg->rope_base != 0.0f) orc_model_rope(m, cfg->max_seq, cfg->rope_base);
    return m;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    free(m->arena); free(m->layers); free(m->rope_cos); free(m->rope_sin); free(m);
}

int orc_model_n_params(const orc_model *m) { return 1 + NPL * m->cfg.L + 2; }

float *orc_model_param(orc_model *m, int i, long long *numel) {
    long long V = m->cfg.V, D = m->cfg.D, F = m->cfg.F;
    if (i == 0) { *numel = V * D; return m->embed; }
    i -= 1;
    if (i < NPL * m->cfg.L) {
        orc_layer *ly = &m->layers[i / NPL];
        switch (i % NPL) {
        case 0:  *numel = D * 3 * D; return ly->wqkv;
        case 1:  *numel = 3 * D;     return ly->bqkv;
        case 2:  *numel = D * D;     return ly->wo;
        case 3:  *numel = D;         return ly->bo;
        case 4:  *numel = D;         return ly->g_attn;
        case 5:  *numel = D;         return ly->g_ffn;
        case 6:  *numel = D * F;     return ly->wg;
        case 7:  *numel = F;         return ly->bg;
        case 8:  *numel = D * F;     return ly->wu;
        case 9:  *numel = F;         return ly->bu;
        case 10: *numel = F * D;     return ly->wd;
        default: *numel = D;         return ly->bd;
        }
    }
    i -= NPL * m->cfg.L;
    if (i == 0) { *numel = D; return m->g_final; }
    *numel = V; return m->lm_bias;
}

static int is_gamma(const orc_model *m, int i) {
    if (i == 0) return 0;
    i -= 1;
    if (i < NPL * m->cfg.L) return (i % NPL) == 4 || (i % NPL) == 5;
    return (i - NPL * m->cfg.L) == 0;
}

/* tensor_uniform (tensor.c:154-162) */
static void fill_uniform(float *p, long long n, float bound) {
    for (long long i = 0; i < n; i++)
        p[i] = (2.0f * orc_rng_uniform(&g_rng) - 1.0f) * bound;
}

void orc_model_init_create(orc_model *m, uint64_t seed) {
    orc_rng_seed(&g_rng, seed);                                     /* dnn_seed, rng.c:76-78 */
    int D = m->cfg.D, F = m->cfg.F, V = m->cfg.V;
    fill_uniform(m->embed, (long long)V * D, 1.0f / sqrtf((float)D)); /* nn.c:177-191 */
    for (int l = 0; l < m->cfg.L; l++) {                            /* transformer.c:116-147 */
        orc_layer *ly = &m->layers[l];
        float bD = 1.0f / sqrtf((float)D), bF = 1.0f / sqrtf((float)F);
        fill_uniform(ly->wqkv, (long long)D * 3 * D, bD); fill_uniform(ly->bqkv, 3 * D, bD);
        fill_uniform(ly->wo, (long long)D * D, bD);       fill_uniform(ly->bo, D, bD);
        fill_uniform(ly->wg, (long long)D * F, bD);       fill_uniform(ly->bg, F, bD);
        fill_uniform(ly->wu, (long long)D * F, bD);       fill_uniform(ly->bu, F, bD);
        fill_uniform(ly->wd, (long long)F * D, bF);       fill_uniform(ly->bd, D, bF);
        for (int i = 0; i < D; i++) ly->g_attn[i] = ly->g_ffn[i] = 1.0f;
    }
    for (int i = 0; i < D; i++) m->g_final[i] = 1.0f;
    memset(m->lm_bias, 0, sizeof(float) * (size_t)V);               /* gpt.c:57 */
}

void orc_model_init_synthetic(orc_model *m, float std) {
    int n = orc_model_n_params(m);
    for (int i = 0; i < n; i++) {
        if (is_gamma(m, i)) continue;
        long long ne;
        float *p = orc_model_param(m, i, &ne);
        for (long long j = 0; j < ne; j++) p[j] = orc_rng_normal(&g_rng) * std;
    }
}

void orc_model_init_gpt2(orc_model *m) {                             /* gpt.c:431-477 */
    float std = 1.0f / sqrtf((float)m->cfg.D);
    float rstd = std / sqrtf(2.0f * (float)m->cfg.L);
    long long D = m->cfg.D, F = m->cfg.F;
    for (long long i = 0; i < (long long)m->cfg.V * D; i++) m->embed[i] = orc_rng_normal(&g_rng) * std;
    for (int l = 0; l < m->cfg.L; l++) {     /* module walk: qkv, out, ffn.{gate,up,down} */
        orc_layer *ly = &m->layers[l];
        for (long long i = 0; i < D * 3 * D; i++) ly->wqkv[i] = orc_rng_normal(&g_rng) * std;
        memset(ly->bqkv, 0, sizeof(float) * 3 * D);
        for (long long i = 0; i < D * D; i++) ly->wo[i] = orc_rng_normal(&g_rng) * rstd;
        memset(ly->bo, 0, sizeof(float) * D);
        for (long long i = 0; i < D * F; i++) ly->wg[i] = orc_rng_normal(&g_rng) * std;
        memset(ly->bg, 0, sizeof(float) * F);
        for (long long i = 0; i < D * F; i++) ly->wu[i] = orc_rng_normal(&g_rng) * std;
        memset(ly->bu, 0, sizeof(float) * F);
        for (long long i = 0; i < F * D; i++) ly->wd[i] = orc_rng_normal(&g_rng) * rstd;
        memset(ly->bd, 0, sizeof(float) * D);
    }
    memset(m->lm_bias, 0, sizeof(float) * (size_t)m->cfg.V);   /* tied lm_head: bias only */
}

void orc_model_rope(orc_model *m, int max_seq, float base) {  /* rope.c:148-171 */
    int dim = m->cfg.dk, half = dim / 2;
    if (base == 0.0f) base = 10000.0f;
    free(m->rope_cos); free(m->rope_sin);
    m->rope_cos = calloc((size_t)max_seq * half, sizeof(float));
    m->rope_sin = calloc((size_t)max_seq * half, sizeof(float));
    for (int k = 0; k < half; k++) {
        float theta = powf(base, -2.0f * k / (float)dim);
        for (int n = 0; n < max_seq; n++) {
            float angle = (float)n * theta;
            m->rope_cos[n * half + k] = cosf(angle);
            m->rope_sin[n * half + k] = sinf(angle);
        }
    }
    m->cfg.max_seq = max_seq;
    m->cfg.rope_base = base;
}

/* ----------------------------------------------------------------- ops */

/* tensor_matmul_add, NO_CBLAS N-D branch (ops_matrix.c:1124-1151).
 * y[i][j] = (sum_k a[i][k]*w[k][j]) + b[j], k ascending, no contraction.
 * trans_b: w is [N][K] and the product walks w[j][k] (ops_matrix.c:1124-1132). */
void orc_matmul_add(const float *a, const float *w, const float *b, float *y,
                    int M, int K, int N, int trans_b) {
    for (int i = 0; i < M; i++) {
        const float *ai = a + (long long)i * K;
        float *yi = y + (long long)i * N;
        if (trans_b) {
            for (int j = 0; j < N; j++) {
                const float *wj = w + (long long)j * K;
                float sum = 0.0f;
                for (int k = 0; k < K; k++) sum += ai[k] * wj[k];
                yi[j] = sum + b[j];
            }
        } else {
            /* every yi[j] accumulates a[k]*w[k][j] for k = 0..K-1 in order */
            for (int j = 0; j < N; j++) yi[j] = 0.0f;
            for (int k = 0; k < K; k++) {
                const float ak = ai[k];
                const float *wk = w + (long long)k * N;
                for (int j = 0; j < N; j++) yi[j] += ak * wk[j];
            }
            for (int j = 0; j < N; j++) yi[j] = yi[j] + b[j];
        }
    }
}

/* tensor_rms_norm (norm.c:404-495), x86 branch.  The sum of squares keeps the
 * reference's `omp simd reduction` loop so gcc vectorises it the same way. */
void orc_rms_norm(const float *x, const float *w, float *y, int n, int d, float eps) {
    for (int s = 0; s < n; s++) {
        const float *xs = x + (long long)s * d;
        float sum_x2 = 0.0f;
        #pragma omp simd reduction(+:sum_x2)
        for (int j = 0; j < d; j++) sum_x2 += xs[j] * xs[j];
        float mean_x2 = sum_x2 * (1.0f / (float)d);
        float rs = 1.0f / sqrtf(mean_x2 + eps);
        float *ys = y + (long long)s * d;
        #pragma omp simd
        for (int j = 0; j < d; j++) {
            float t = xs[j] * rs;
            ys[j] = t * (w ? w[j] : 1.0f);
        }
    }
}

/* _rope_apply (rope.c:20-35): interleaved pairs (2k, 2k+1). c/s point at the
 * table row for each row's position; rows advance by d floats, tables by d/2. */
void orc_rope_rows(float *x, int n_rows, int d, const float *c, const float *s) {
    int half = d / 2;
    for (int r = 0; r < n_rows; r++) {
        float *row = x + (long long)r * d;
        const float *cr = c + (long long)r * half, *sr = s + (long long)r * half;
        for (int k = 0; k < half; k++) {
            float e = row[2 * k], o = row[2 * k + 1];
            row[2 * k]     = e * cr[k] - o * sr[k];
            row[2 * k + 1] = e * sr[k] + o * cr[k];
        }
    }
}

/* simd_swiglu_fwd scalar branch (simd.h:394-397). */
void orc_swiglu(const float *g, const float *u, float *y, int n) {
    for (int i = 0; i < n; i++) y[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* One query row of the cached attention (transformer.c:290-297, 353-390): the
 * first S keys are visible.  Masked keys of the reference (-INF scores) add
 * exactly 0 to se and to every o[c], so only the visible prefix is walked. */
void orc_attend_row(const float *q, const float *k, const float *v, int S, int dk,
                    int row_stride, float *scores, float *o) {
    float scale = 1.0f / sqrtf((float)dk);
    for (int j = 0; j < S; j++) {
        const float *kj = k + (long long)j * row_stride;
        float sum = 0.0f;
        for (int kk = 0; kk < dk; kk++) sum += q[kk] * kj[kk];
        scores[j] = sum * scale;
    }
    float mx = -INFINITY, se = 0.0f;
    for (int j = 0; j < S; j++) {
        float old_mx = mx;
        if (scores[j] > mx) mx = scores[j];
        if (mx != old_mx) se *= expf(old_mx - mx);
        se += expf(scores[j] - mx);
    }
    float inv_se = 1.0f / se;
    for (int j = 0; j < S; j++) scores[j] = expf(scores[j] - mx) * inv_se;
    for (int c = 0; c < dk; c++) {
        float sum = 0.0f;
        for (int j = 0; j < S; j++) sum += scores[j] * v[(long long)j * row_stride + c];
        o[c] = sum;
    }
}

int orc_argmax(const float *logits, int n) {      /* gpt.c:220-230 */
    int best = 0;
    float best_val = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > best_val) { best_val = logits[i]; best = i; }
    return best;
}

void orc_embed(const orc_model *m, const int *ids, int N, float *x) {  /* embedding.c:79-84 */
    int D = m->cfg.D;
    for (int i = 0; i < N; i++) {
        assert(ids[i] >= 0 && ids[i] < m->cfg.V);
        memcpy(x + (long long)i * D, m->embed + (long long)ids[i] * D, sizeof(float) * D);
    }
}

void orc_head(const orc_model *m, const float *x, int N, float *logits) {
    int D = m->cfg.D;
    float *h = malloc(sizeof(float) * (size_t)N * D);
    orc_rms_norm(x, m->g_final, h, N, D, 1e-5f);                        /* gpt.c:357 */
    orc_matmul_add(h, m->embed, m->lm_bias, logits, N, D, m->cfg.V, 1);  /* gpt.c:117-122 */
    free(h);
}

/* --------------------------------------------------------------- state */

orc_state *orc_state_create(const orc_model *m, int max_seq) {
    orc_state *s = calloc(1, sizeof(*s));
    s->m = m;
    s->max_seq = max_seq;
    size_t kv = (size_t)m->cfg.L * m->cfg.H * max_seq * m->cfg.dk;
    s->k = calloc(kv, sizeof(float));
    s->v = calloc(kv, sizeof(float));
    return s;
}

void orc_state_free(orc_state *s) {
    if (!s) return;
    free(s->k); free(s->v); free(s->scratch); free(s);
}

void orc_state_reset(orc_state *s) { s->seq_len = 0; }

void orc_state_kv(const orc_state *s, int layer, int which, int len, float *out) {
    const int H = s->m->cfg.H, dk = s->m->cfg.dk;
    assert(len <= s->seq_len);
    const float *src = (which ? s->v : s->k) + (size_t)layer * H * s->max_seq * dk;
    for (int h = 0; h < H; h++)
        memcpy(out + (size_t)h * len * dk, src + (size_t)h * s->max_seq * dk, sizeof(float) * (size_t)len * dk);
}

/* transformer_block_forward_cached_ex (transformer.c:211-416) for every layer. */
void orc_forward_cached(orc_state *st, float *x, int N, int mode, int prefix_len) {
    const orc_model *m = st->m;
    const int D = m->cfg.D, H = m->cfg.H, dk = m->cfg.dk, F = m->cfg.F;
    const int old = st->seq_len, S = old + N;
    assert(S <= st->max_seq && "kv cache full (transformer.c:55-56)");
    assert(!(mode == 1 && old != 0) && "prefix-LM prefill needs an empty cache");
    if (m->rope_cos) assert(S <= m->cfg.max_seq && "RoPE table too short");

    float *h = malloc(sizeof(float) * (size_t)N * D);
    float *qkv = malloc(sizeof(float) * (size_t)N * 3 * D);
    float *q = malloc(sizeof(float) * (size_t)N * dk);
    float *att = malloc(sizeof(float) * (size_t)N * D);
    float *proj = malloc(sizeof(float) * (size_t)N * D);
    float *g = malloc(sizeof(float) * (size_t)N * F);
    float *u = malloc(sizeof(float) * (size_t)N * F);
    float *sc = malloc(sizeof(float) * (size_t)S);

    for (int l = 0; l < m->cfg.L; l++) {
        const orc_layer *ly = &m->layers[l];
        float *kc = st->k + (size_t)l * H * st->max_seq * dk;
        float *vc = st->v + (size_t)l * H * st->max_seq * dk;

        orc_rms_norm(x, ly->g_attn, h, N, D, 1e-5f);                  /* :232 */
        orc_matmul_add(h, ly->wqkv, ly->bqkv, qkv, N, D, 3 * D, 0);   /* :235 */

        for (int hh = 0; hh < H; hh++) {
            /* split (multihead.c:240-263): Q cols [0,D), K [D,2D), V [2D,3D) */
            float *kh = kc + (size_t)hh * st->max_seq * dk;
            float *vh = vc + (size_t)hh * st->max_seq * dk;
            for (int i = 0; i < N; i++) {
                const float *row = qkv + (size_t)i * 3 * D;
                memcpy(q + (size_t)i * dk, row + hh * dk, sizeof(float) * dk);
                memcpy(kh + (size_t)(old + i) * dk, row + D + hh * dk, sizeof(float) * dk);
                memcpy(vh + (size_t)(old + i) * dk, row + 2 * D + hh * dk, sizeof(float) * dk);
            }
            if (m->rope_cos) {                                         /* :240-247 */
                const float *c = m->rope_cos + (size_t)old * (dk / 2);
                const float *s = m->rope_sin + (size_t)old * (dk / 2);
                orc_rope_rows(q, N, dk, c, s);
                orc_rope_rows(kh + (size_t)old * dk, N, dk, c, s);     /* K stored post-RoPE */
            }
            for (int i = 0; i < N; i++) {                              /* :274-397 */
                int gq = old + i;
                int vis = (mode == 1) ? ((gq < prefix_len) ? prefix_len : gq + 1) : gq + 1;
                if (vis > S) vis = S;
                orc_attend_row(q + (size_t)i * dk, kh, vh, vis, dk, dk, sc,
                               att + (size_t)i * D + hh * dk);          /* merge_heads layout */
            }
        }
        orc_matmul_add(att, ly->wo, ly->bo, proj, N, D, D, 0);          /* :405 */
        for (long long i = 0; i < (long long)N * D; i++) x[i] = x[i] + proj[i];   /* :408 */
        orc_rms_norm(x, ly->g_ffn, h, N, D, 1e-5f);                     /* :411 */
        orc_matmul_add(h, ly->wg, ly->bg, g, N, D, F, 0);               /* nn.c:67 */
        orc_matmul_add(h, ly->wu, ly->bu, u, N, D, F, 0);               /* nn.c:70 */
        orc_swiglu(g, u, g, N * F);                                     /* nn.c:73 */
        orc_matmul_add(g, ly->wd, ly->bd, proj, N, F, D, 0);            /* nn.c:76 */
        for (long long i = 0; i < (long long)N * D; i++) x[i] = x[i] + proj[i];   /* :415 */
    }
    st->seq_len = S;
    free(h); free(qkv); free(q); free(att); free(proj); free(g); free(u); free(sc);
}

/* decoder_lm_generate, use_cache=1, greedy (gpt.c:258-375). */
int orc_generate(const orc_model *m, const int *prompt, int P, int max_new,
                 int eos, int *out, float *logits) {
    const int D = m->cfg.D, V = m->cfg.V;
    int max_len = P + max_new;
    orc_state *st = orc_state_create(m, max_len);
    float *x = malloc(sizeof(float) * D);
    float *lg = malloc(sizeof(float) * V);
    memcpy(out, prompt, sizeof(int) * P);
    int cur = P, n_logit = 0;
    for (int p = 0; p < P; p++) {                    /* prompt one token at a time (:306-344) */
        orc_embed(m, &out[p], 1, x);
        orc_forward_cached(st, x, 1, 0, 0);
        if (p == P - 1) {
            orc_head(m, x, 1, lg);
            if (logits) memcpy(logits + (size_t)n_logit++ * V, lg, sizeof(float) * V);
            int id = orc_argmax(lg, V);
            out[cur++] = id;
            if (id == eos) goto done;
        }
    }
    while (cur < max_len) {                           /* :347-375 */
        orc_embed(m, &out[cur - 1], 1, x);
        orc_forward_cached(st, x, 1, 0, 0);
        orc_head(m, x, 1, lg);
        if (logits) memcpy(logits + (size_t)n_logit++ * V, lg, sizeof(float) * V);
        int id = orc_argmax(lg, V);
        out[cur++] = id;
        if (id == eos) break;
    }
done:
    free(x); free(lg);
    orc_state_free(st);
    return cur;
}

/* decoder_lm_forward without cache: the full-sequence block
 * (transformer.c:151-201) with tensor_attention_ex's triangular forward
 * (attention.c:259-380).  Row i sees keys [0, i]; its scores, softmax and P.V
 * are the same float sequences as the cached path's, so one cached pass over
 * the N rows from an empty cache is this forward. */
void orc_forward_full(const orc_model *m, const int *ids, int N, float *logits) {
    orc_state *st = orc_state_create(m, N);
    float *x = malloc(sizeof(float) * (size_t)N * m->cfg.D);
    orc_embed(m, ids, N, x);
    orc_forward_cached(st, x, N, 0, 0);
    orc_head(m, x, N, logits);
    free(x);
    orc_state_free(st);
}

/* FNV-1a 64 over raw bytes: the fixture files identify float buffers by it. */
uint64_t orc_fnv(const void *p, size_t n) {
    const unsigned char *b = p;
    uint64_t h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}

/* RoPE tables of the model (NULL when disabled) and their row count. */
const float *orc_model_rope_cos(const orc_model *m) { return m->rope_cos; }
const float *orc_model_rope_sin(const orc_model *m) { return m->rope_sin; }
int orc_model_rope_rows(const orc_model *m) { return m->rope_cos ? m->cfg.max_seq : 0; }
