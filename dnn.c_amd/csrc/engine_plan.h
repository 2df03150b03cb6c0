// engine_plan.h -- launch planning of the batched engine's decode-shape GEMMs
// (workgroups per column tile, row tiles per workgroup, wavefronts splitting
// K), the split-K buffers they need, and the decode attention's wavefronts,
// key splits and speculative loads.  Plain C++ (no HIP): the engine and a
// CPU test of the plans include it.  Internal: not part of the public headers.
#pragma once
#include <algorithm>
#include <cstddef>
#include <cstdlib>

namespace dnnhip {

constexpr int CNT_GEMM = 4096;           // last-arriver counters of GEMM column tiles
constexpr int PLAN_MAX_ROWS = 64;        // rows of a session (MAX_ROWS)

// k-steps per wavefront the decode GEMM is built for (pick_ks chooses among
// them), and those instantiated for eight and four wavefronts per workgroup
// (gemm_decode_mt's launch switch)
constexpr int GEMM_KPW[] = {12, 8, 6, 4, 3, 2};
constexpr int GEMM_KPW_KW8[] = {2, 3, 4, 6, 8};
constexpr int GEMM_KPW_KW4[] = {2, 3, 4, 6, 8, 12};

// Workgroups a decode GEMM without rms_norm is split towards (read once, so
// the partial buffers sized at engine creation match every launch);
// DNN_HIP_KS_FILL overrides.  Measured at 32 rows (C3): 64 -> 66.1k tokens/s,
// 128 / 192 / 256 / 384 -> 64.4k / 64.3k / 63.8k / 63.2k (out_proj split over
// 2..4 workgroups per tile); 8 rows: 192 0.6% slower; 64 rows within noise.
inline int ks_fill() {
    static const int v = [] {
        const char *e = getenv("DNN_HIP_KS_FILL");
        return e ? std::max(1, atoi(e)) : 64;
    }();
    return v;
}

// Split of a decode GEMM: k-steps per wavefront (kpw, one of GEMM_KPW) and
// workgroups per column tile (ks), K/16 = 4 * ks * kpw.  A wavefront holds all
// of its A and W loads in registers at once, which bounds kpw by the row tiles
// per workgroup (mt_max, 0 = all); a GEMM without rms_norm is split further
// until it has ks_fill() workgroups (the split's partials and last-arriver cost
// more than the extra parallelism gains below that).
inline int pick_ks(int ntiles, int K, int M, bool norm, int mt_max = 0) {
    const int nks = K / 16, tiles_m = (M + 15) / 16;
    const int mt = mt_max > 0 && tiles_m > mt_max ? mt_max : tiles_m;
    const int row_groups = (tiles_m + mt - 1) / mt;
    static const int lim_norm[4] = {19, 14, 11, 9}, lim_plain[4] = {28, 19, 14, 11};
    const int lim = (norm ? lim_norm : lim_plain)[mt - 1];
    int best = 0;
    for (int kpw : GEMM_KPW) {
        if (kpw > lim || nks % (4 * kpw)) continue;
        const int ks = nks / (4 * kpw);
        if (ks > 8) break;
        best = ks;
        if (norm || ntiles * ks * row_groups >= ks_fill()) break;
    }
    return best;
}

// Wavefronts splitting K in a decode GEMM workgroup: 8 where each then still
// holds 2 to 8 k-blocks (half the MFMA chain and loads per wavefront of 4:
// C3 60.4k -> 61.9k, C5 142k -> 149k tokens/s), else 4; DNN_HIP_GEMM_KW=4
// keeps 4.
inline int decode_kw(int nks, int ks) {
    static const int forced = [] {
        const char *e = getenv("DNN_HIP_GEMM_KW");
        return e ? atoi(e) : 0;
    }();
    const bool eight_ok = nks % (8 * ks) == 0 && nks / (8 * ks) >= 2 && nks / (8 * ks) <= 8;
    return forced != 4 && eight_ok ? 8 : 4;
}

// Row tiles per workgroup of the decode QKV and gate/up GEMMs (rms_norm fused,
// not split over K): one for QKV, so every 16 rows launch the column tiles'
// workgroups again; one for gate/up from 33 rows on, all rows below (measured:
// 64 rows 149k -> 179k tokens/s with the down GEMM's single tile, 32 rows QKV
// +0.5%, gate/up at one tile 1% slower).  DNN_HIP_QKV_MT / DNN_HIP_GU_MT
// override (0: all rows).
inline int norm_mt(const char *env, int M, bool qkv) {
    if (const char *v = getenv(env)) return atoi(v);
    return qkv || (M + 15) / 16 > 2 ? 1 : 0;
}

// Row tiles per workgroup of the decode down GEMM (one, as out_proj: 64 rows
// 160k -> 169k tokens/s, 32 rows unchanged) and lm_head GEMM (all rows: one
// per workgroup was slower at 32 and 64 rows); DNN_HIP_DOWN_MT /
// DNN_HIP_HEAD_MT override (0: all rows).
inline int plain_mt(const char *env, int dflt) {
    const char *v = getenv(env);
    return v ? atoi(v) : dflt;
}

// Split-K partial pairs a decode GEMM of these dimensions needs.
inline size_t part_pairs_for(int N, int K, int M, bool norm, int mt_max = 0) {
    const int ntn = (N + 15) / 16, ks = pick_ks(ntn, K, M, norm, mt_max);
    return ks > 1 ? (size_t)ks * M * N + (size_t)ntn * ks * M : 0;
}

// Row tiles per workgroup (mt_max) of each decode-shape GEMM, as the launches
// use them: the layer GEMMs of decode steps, and the lm_head of decode steps
// (head_decode) or of prefill / dnn_hip_head_forward (all rows).
struct MtPlan {
    int qkv, out, gu, down, head;
};
inline MtPlan mt_plan(int M, bool head_decode) {
    MtPlan p;
    p.qkv = norm_mt("DNN_HIP_QKV_MT", M, true);
    p.out = 1;                       // out_proj: one 16-row tile per workgroup (more, lighter workgroups)
    p.gu = norm_mt("DNN_HIP_GU_MT", M, false);
    p.down = plain_mt("DNN_HIP_DOWN_MT", 1);
    p.head = head_decode ? plain_mt("DNN_HIP_HEAD_MT", 0) : 0;
    return p;
}

// Split-K partial pairs the engine needs for a model: the largest need of any
// decode-shape GEMM launch (QKV, out_proj, gate/up, down, lm_head) at any row
// count, for decode steps and for prefill / head calls.
// Wavefronts per workgroup of the decode attention (attn_kernel<AW>) for M
// rows of H heads: eight where there are few (row, head) pairs, else four.
inline int attn_waves(int M, int H) { return M * H <= 128 ? 8 : 4; }

// Workgroups per (row, head) of the decode attention over histories of up to
// S_max keys: one where the rows and heads alone fill the chip, else the fewest
// that leave each wavefront at most two 64-key chunks (a split's merge -- the
// partials, the counter and the last arriver's reload -- costs more than a
// wider launch gains: measured on 8 rows of 32..1087 keys); at most 8.  req > 0
// (DNN_HIP_ATT_SPLITS) fixes it.
inline int attn_splits_for(int req, int M, int H, int S_max) {
    if (req > 0) return std::min(8, req);
    if (M * H >= 256) return 1;
    const int aw = attn_waves(M, H), nch = (S_max + 63) / 64;
    return std::max(1, std::min(8, (nch + 2 * aw - 1) / (2 * aw)));
}

// Decode-attention wavefronts (of aw per workgroup, ns key splits per head)
// that load their first chunk before the row's length is known: the leading
// ones whose first chunk (64 keys of split 0) at least 3/4 of the call's
// (row, step) pairs have -- pos[b] is row b's position at the call's first
// step -- at least one, and at least four of eight (few (row, head) pairs, so
// keys fetched for nothing cost little).  DNN_HIP_ATT_SPEC=n fixes it (tuning;
// read at every call).
inline int attn_spec(int aw, int ns, int B, int n_steps, const int *pos) {
    int spec = aw == 8 ? 4 : 1;
    for (int w = spec; w < aw; w++) {
        const long long keys = 64LL * ns * w;
        long long have = 0;
        for (int b = 0; b < B; b++) {
            const long long first = keys - pos[b];      // steps t with pos + t + 1 > keys: t >= first
            have += std::max(0LL, (long long)n_steps - std::max(0LL, first));
        }
        if (4 * have < 3LL * B * n_steps) break;
        spec = w + 1;
    }
    if (const char *v = getenv("DNN_HIP_ATT_SPEC")) spec = std::max(1, std::min(aw, atoi(v)));
    return spec;
}

inline size_t engine_part_need(int D, int F, int V, int ldD, int ldF) {
    size_t need = 1;
    for (int rows = 1; rows <= PLAN_MAX_ROWS; rows++)
        for (int hd = 0; hd < 2; hd++) {
            const MtPlan p = mt_plan(rows, hd != 0);
            const size_t n[5] = {part_pairs_for(3 * D, ldD, rows, true, p.qkv),
                                 part_pairs_for(D, ldD, rows, false, p.out),
                                 part_pairs_for(2 * F, ldD, rows, true, p.gu),
                                 part_pairs_for(D, ldF, rows, false, p.down),
                                 part_pairs_for(V, ldD, rows, true, p.head)};
            for (size_t v : n) need = std::max(need, v);
        }
    return need;
}

}  // namespace dnnhip
