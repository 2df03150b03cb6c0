// decode_kernel_body.h -- the persistent decode kernel decode_v3<NB, DC, BF>
// (described in decode_kernel.hip); included by the translation units that
// instantiate it (fp32 weights in decode_kernel.hip, bf16 in
// decode_kernel_bf16.hip) so the two compile in parallel.
#pragma once
#include "decode_device.h"

namespace dnnhip {

// DNNHIP_TRACE (timing builds only, never the product): thread 0 of every
// workgroup stamps s_memrealtime at the phase boundaries of one chosen step
// into trace[workgroup][layer (L = head)][event].
#ifdef DNNHIP_TRACE
constexpr int TRACE_L = 33, TRACE_E = 16;
__device__ unsigned long long g_trace[256 * TRACE_L * TRACE_E];
__device__ int g_trace_step;
#define TRACE_EV(L_, EV)                                                                              \
    do {                                                                                              \
        if (tid == 0 && t == g_trace_step)                                                            \
            g_trace[((size_t)g0 * TRACE_L + (L_)) * TRACE_E + (EV)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define TRACE_EV(L_, EV) \
    do {                 \
    } while (0)
#endif

// Attention rows AS from the split records of one layer (heads split over ns
// workgroups): record r = (b*H + h)*ns + s carries O_s = sum_j e^(s_j - m_s) v_j
// (DK values) and (m_s, l_s = sum_j e^(s_j - m_s)); the row of head (b, h) is
// sum_s e^(m_s - M) O_s / sum_s e^(m_s - M) l_s with M = max_s m_s -- the
// softmax-weighted sum of transformer.c:349-397, merged from key ranges.
// Wavefront w takes heads w, w + 8, ... (at most ATT_SPLIT_HEADS / 8 of them),
// every record of its heads polled in one pass.
__device__ __forceinline__ void stage_att_split(float *as, int ld, int nh, int H, int ns, size_t ao, size_t aml,
                                                rsrc_t xa, unsigned tag, int wid, int lane, Waiter &wt) {
    constexpr int HPW = ATT_SPLIT_HEADS / WPB;
    u2 o[HPW][ATT_SPLIT_MAX], ml[HPW];
    wt.reset();
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < HPW; i++) {
            const int hb = wid + i * WPB;
            if (hb >= nh) continue;
#pragma unroll
            for (int sp = 0; sp < ATT_SPLIT_MAX; sp++) {
                if (sp >= ns) continue;
                o[i][sp] = __builtin_amdgcn_raw_buffer_load_b64(
                    xa, (unsigned)((ao + ((size_t)hb * ns + sp) * DK + lane) * 8), 0, CP_SC1);
                ok &= o[i][sp].y == tag;
            }
            const int li = lane < 2 * ns ? lane : 0;
            ml[i] = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)((aml + (size_t)hb * ns * 2 + li) * 8), 0, CP_SC1);
            ok &= ml[i].y == tag;
        }
        if (__all(ok) || !wt.again()) break;
    }
#pragma unroll
    for (int i = 0; i < HPW; i++) {
        const int hb = wid + i * WPB;
        if (hb >= nh) continue;
        const float mv = as_float(ml[i].x);
        float M = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < ATT_SPLIT_MAX; sp++)
            if (sp < ns) M = fmaxf(M, bcast(mv, 2 * sp));
        float O = 0.f, den = 0.f;
#pragma unroll
        for (int sp = 0; sp < ATT_SPLIT_MAX; sp++) {
            if (sp >= ns) continue;
            const float m = bcast(mv, 2 * sp);
            const float f = m == -INFINITY ? 0.f : expf(m - M);
            O += f * as_float(o[i][sp].x);
            den += f * bcast(mv, 2 * sp + 1);
        }
        const int b = hb / H, h = hb - b * H;
        as[b * ld + h * DK + lane] = O / den;
    }
}

// The decode loop of one session on workgroups g0 = 0 .. G-1.
//
// Every workgroup has one role for the whole launch and runs its own copy of
// the step / layer loop: QKV and out_proj (phases A and C), attention (B), the
// gate/up GEMV (D) or the down GEMV (E); the attention and D workgroups also
// run the lm_head (F), and all of them reduce the argmax (G).  No workgroup
// runs two consecutive phases of the layer chain A -> B -> C -> D -> E -> A'.
// A CU's vector-memory requests are served in issue order, so a workgroup that
// stored a phase's outputs and then polled the next phase's inputs would wait
// behind its own weight loads; with roles, a workgroup stores its outputs,
// then issues the weight loads of its next phase, and those land while the
// other roles run.  Rounds of a role's GEMV: unit u of round k on role-local
// workgroup r is (k * n_role + r) * WPB + wid, so a workgroup's outputs of a
// round are contiguous; the first PH rounds stay in registers ahead of the
// phase, later ones load in batches of PH.
template <int NB, int DC, bool BF>
__device__ __forceinline__ void decode_v3_body(const DecodeArgs &a, const int G, const int g0) {
    extern __shared__ float smem[];
    int *s_tok = reinterpret_cast<int *>(smem);                 // [MAXB]
    int *s_pos = s_tok + MAXB;                                  // [MAXB]
    int *s_done = s_pos + MAXB;                                 // [MAXB]
    float *s_bv = reinterpret_cast<float *>(s_done + MAXB);     // [WPB][MAXB]
    int *s_bi = reinterpret_cast<int *>(s_bv + WPB * MAXB);     // [WPB][MAXB]
    float *s_part = reinterpret_cast<float *>(s_bi + WPB * MAXB);   // [WPB][DK + 2]
    float *s_out = s_part + WPB * (DK + 2);                     // [PU][WPB][2 * MAXB]
    float *s_qe = s_out + PU * WPB * 2 * MAXB;                  // [WPB][DK + CPW * CH]
    const int ldD = a.ldD, ldF = a.ldF;
    float *xs = smem + (LDS_HEAD_WORDS + 3) / 4 * 4;            // [NB][ldD] layer input (raw)
    float *as = xs + NB * ldD;                                  // [NB][ldD] attention output
    float *x1s = as + NB * ldD;                                 // [NB][ldD] X1 (raw)
    float *acts = x1s + NB * ldD;                               // [NB][ldF] SwiGLU output
    constexpr int PH = hold_rounds(NB, DC);                     // rounds held in registers (<= PU)

    const int tid = threadIdx.x;
    int lane = tid & (WAVE - 1);
    const int wid = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int B = a.B, D = a.D, H = a.H, F = a.F, V = a.V;
    const int nrows = B < NB ? B : NB;
    const int ns = a.ex.ns > 1 ? a.ex.ns : 1;                  // workgroups per (row, head)
    Waiter wt{a.err};

    const size_t kv_head = (size_t)DK * a.max_seq;              // floats per (layer, row, head)
    const rsrc_t rw = buf(a.wts, a.wts_bytes);
    // weight matrices: the fp32 arena, or its bf16 copy at the same element
    // offsets (biases, gammas and the embedding gather always read the fp32 arena)
    const rsrc_t rm = BF ? buf(a.wts16, a.wts_bytes / 2) : rw;
    const rsrc_t xa = buf(a.xa, a.ex.total(a.L) * 8);
    const size_t kv_bytes = ((size_t)a.L * B * H * kv_head + (size_t)CH * DK) * 4;   // incl. the padding
    const rsrc_t rk = buf(a.kc, kv_bytes);
    const rsrc_t rv = buf(a.vc, kv_bytes);
    const size_t sin_off = (size_t)a.rope_rows * (DK / 2) * 4;      // bytes
    const rsrc_t rrope = buf(a.rope, a.rope ? 2 * sin_off : 0);
    const size_t xstride = a.ex.per_row();
    const float scale = 1.0f / sqrtf((float)DK);

    // roles: [0, n_ac) A+C, then n_d D, n_e E, the rest attention; the lm_head
    // runs on the D workgroups, then the E ones (index fi of nF)
    const int nAC = a.n_ac, nDD = a.n_d, nEE = a.n_e;
    const int nAT = G - nAC - nDD - nEE;
    const int nF = nDD + nEE;
    int role, r0;
    if (g0 < nAC) { role = R_AC; r0 = g0; }
    else if (g0 < nAC + nDD) { role = R_D; r0 = g0 - nAC; }
    else if (g0 < nAC + nDD + nEE) { role = R_E; r0 = g0 - nAC - nDD; }
    else { role = R_ATT; r0 = g0 - nAC - nDD - nEE; }
    const int fi = role == R_D ? r0 : nDD + r0;                 // lm_head index (D and E roles)

    for (int i = tid; i < NB * (3 * ldD + ldF); i += BLOCK) xs[i] = 0.f;
    for (int b = tid; b < MAXB; b += BLOCK) {
        s_pos[b] = b < B ? a.pos[b] : 0;
        s_done[b] = 0;
        s_tok[b] = 0;
    }
    __syncthreads();
    // every row must have room for the launch's steps (the host checks this
    // where it knows the lengths; callers that keep them on the device rely on
    // this): otherwise every workgroup leaves before touching anything, and
    // the launch reports error bit 1
    bool room = true;
    for (int b = 0; b < B; b++) room &= s_pos[b] >= 0 && s_pos[b] + a.n_steps <= a.seq_limit;
    if (!room) {
        if (g0 == 0 && tid == 0) {
            atomicOr(a.err, 2);
            *a.steps_done = 0;
        }
        return;
    }

    int t = 0;
    bool pre = false;                                            // A+C role: layer 0's units held

    // attention workgroups without a record (other than the reducer) have
    // nothing to do: nothing waits for them
    if (role == R_ATT && r0 >= B * H * ns && r0 != nAT - 1) return;

    auto nrounds = [&](int nu, int n) { return (nu + n * WPB - 1) / (n * WPB); };
    // unit of round k (of kr) on this workgroup: its rounds are consecutive
    // blocks, so all of a workgroup's outputs of a phase are one contiguous
    // range and leave in one store per row instead of one per round
    auto unit = [&](int k, int kr) { return (r0 * kr + k) * WPB + wid; };

    // GEMV units held ahead of their phase: rows (2u, 2u+1) of a [*, ldD]
    // matrix and their biases, or, for an A unit, also the RoPE factors of the
    // rows' positions (lane b < NB: row b)
    RowUnit<2, DC, BF> U[PH];
    float rc[PH], rsn[PH];
    f4 gp[DC];                                                   // gamma of the held phase
    auto load_u = [&](int j, size_t woff, size_t b0, size_t b1) {
        const size_t bo[2] = {b0, b1};
        load_unit<2, DC, BF>(U[j], rw, rm, woff, ldD, bo, lane);
    };
    auto load_a = [&](int j, const LayerOff &w, int u, int dpos) {
        const int n = 2 * u;
        load_u(j, w.wqkv + (size_t)n * ldD, w.bqkv + (size_t)n, w.bqkv + (size_t)n + 1);
        const int sec = n / D, jj = (n - sec * D) % DK;
        rc[j] = 1.f; rsn[j] = 0.f;
        if (sec < 2 && a.rope && lane < NB) {
            const size_t ti = ((size_t)(s_pos[lane < B ? lane : B - 1] + dpos) * (DK / 2) + jj / 2) * 4;
            rc[j] = ld1<0>(rrope, ti);
            rsn[j] = ld1<0>(rrope, sin_off + ti);
        }
    };
    auto load_f = [&](int j, int u) {
        const int v = 2 * u;
        load_u(j, a.embed + (size_t)v * ldD, a.lm_bias + (size_t)v, a.lm_bias + (size_t)v + 1);
    };
    // the first PH rounds of a phase (nu units over n role workgroups)
    auto prefetch = [&](int nu, int n, auto &&load) {
        const int kr = nrounds(nu, n);
#pragma unroll
        for (int j = 0; j < PH; j++)
            if (j < kr) load(j, min(unit(j, kr), nu - 1));
    };
    // Every round of a GEMV phase of 2-row units: per-lane partial sums of
    // the held units (part), one interleaved reduction of all of them, the
    // epilogues (epi) leave the outputs in OUT (rr outputs per unit, rounds
    // consecutive), and wavefront 0 writes the batch's rounds as one block
    // (emit(out, first unit, units)); the trailing barrier also keeps the
    // other wavefronts' next loads behind those stores.
    auto gemv = [&](int nu, int n, int rr, auto &&load, auto &&part, auto &&epi, auto &&emit, int tl, int te) {
        const int kr = nrounds(nu, n);
        const int ostr = WPB * NB * rr;
        for (int k0 = 0; k0 < kr; k0 += PH) {
            if (k0 > 0) {
#pragma unroll
                for (int j = 0; j < PH; j++)
                    if (k0 + j < kr) load(j, min(unit(k0 + j, kr), nu - 1));
            }
            float sm[PH * 2 * NB];
#pragma unroll
            for (int j = 0; j < PH; j++) {
                const int u = unit(k0 + j, kr);
                if (k0 + j < kr && u < nu) {
                    part(j, sm + j * 2 * NB);
                } else {
#pragma unroll
                    for (int i = 0; i < 2 * NB; i++) sm[j * 2 * NB + i] = 0.f;
                }
            }
            wave_sum_n<PH * 2 * NB>(sm);
#pragma unroll
            for (int j = 0; j < PH; j++) {
                const int u = unit(k0 + j, kr);
                if (k0 + j < kr && u < nu) epi(j, u, sm + j * 2 * NB, s_out + j * ostr);
            }
            TRACE_EV(tl, te);
            lds_barrier();
            TRACE_EV(tl, te + 1);
            if (wid == 0) emit(s_out, (r0 * kr + k0) * WPB, min(PH, kr - k0) * WPB);
            lds_barrier();
        }
    };


    // ---- G: the last attention workgroup reduces the lm_head partials (its
    // wavefront w takes rows w, w + 8, ...; first index of the maximum,
    // gpt.c:220-230) and writes each row's token in 8 copies, one per XCD;
    // every workgroup then polls its XCD's copy (one cache line per XCD
    // instead of every partial polled by every workgroup).
    const bool reducer = role == R_ATT && r0 == nAT - 1;
    auto reduce_g = [&](unsigned tag) {
        for (int b = wid; reducer && b < B; b += WPB) {
            float v = -INFINITY;
            int i = 0x7fffffff;
            // every partial in one polling pass (4 per lane)
            for (int gb = 0; gb < nF; gb += 4 * WAVE) {
                u4 q[4];
                wt.reset();
                for (;;) {
                    bool ok = true;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int gg = gb + k * WAVE + lane;
                        const size_t pa = a.ex.amax(a.L, t & 1, b, gg < nF ? gg : 0);
                        q[k] = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)(pa * 8), 0, CP_SC1);
                        ok &= q[k].y == tag && q[k].w == tag;
                    }
                    if (__all(ok) || !wt.again()) break;
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int gg = gb + k * WAVE + lane;
                    const float vv = as_float(q[k].x);
                    const int ii = (int)(unsigned)q[k].z;
                    if (gg < nF && (vv > v || (vv == v && ii < i))) { v = vv; i = ii; }
                }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float vv = __shfl_xor(v, o, WAVE);
                const int ii = __shfl_xor(i, o, WAVE);
                if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
            }
            if (i < 0 || i >= V) i = 0;         // all-NaN row: argmax keeps index 0
            if (lane < 8) put(xa, a.ex.tok(a.L, t & 1, lane, b), __builtin_bit_cast(float, i), tag);
        }
        if (wid == 0) {
            const int b = lane < B ? lane : 0;
            const int i = __builtin_bit_cast(int, poll1(xa, (long)a.ex.tok(a.L, t & 1, g0 & 7, b), tag, wt));
            if (lane < B) {
                s_tok[b] = i;
                s_pos[b] += 1;
                if (a.eos >= 0 && t >= a.n_feed[b] - 1 && i == a.eos) s_done[b] = 1;
                if (g0 == 0) a.ids[(size_t)t * B + b] = i;
            }
        }
        __syncthreads();
        TRACE_EV(a.L, 3);
        if (a.eos >= 0) {
            int all = 1;
            for (int b = 0; b < B; b++) all &= s_done[b];
            if (all) return true;
        }
        return false;
    };

    // ---- F: final rms_norm -> tied lm_head + bias -> this workgroup's argmax
    // partial (D and E roles; their first PH rounds were loaded a phase or
    // more ahead)
    auto lm_head = [&](unsigned tag) {
        TRACE_EV(a.L, 0);
        asm volatile("" : "+v"(lane));
        float bv[NB];
        int bi[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
        const int nu = V / 2;
        stage_rows<NB * 6 / WPB + 1>(xs, ldD, D, nrows, a.ex.x2(a.L - 1, 0), xstride, xa, tag, wid, lane, wt);
        lds_barrier();
        TRACE_EV(a.L, 1);
        float rs[NB];
        rms_lds<NB, DC>(xs, ldD, D, a.eps_final, lane, rs);
        const int kr = nrounds(nu, nF);
        for (int k0 = 0; k0 < kr; k0 += PH) {
            if (k0 > 0) {
#pragma unroll
                for (int j = 0; j < PH; j++)
                    if (k0 + j < kr) load_f(j, min(((k0 + j) * nF + fi) * WPB + wid, nu - 1));
            }
            float sm[PH * 2 * NB];
#pragma unroll
            for (int j = 0; j < PH; j++) {
                const int u = ((k0 + j) * nF + fi) * WPB + wid;
                if (k0 + j < kr && u < nu) {
                    part_lds<2, NB, DC, true>(U[j].w, xs, ldD, rs, gp, lane, sm + j * 2 * NB);
                } else {
#pragma unroll
                    for (int i = 0; i < 2 * NB; i++) sm[j * 2 * NB + i] = 0.f;
                }
            }
            wave_sum_n<PH * 2 * NB>(sm);
#pragma unroll
            for (int j = 0; j < PH; j++) {
                const int u = ((k0 + j) * nF + fi) * WPB + wid, v = 2 * u;
                if (k0 + j >= kr || u >= nu) continue;
                const float *acc = sm + j * 2 * NB;
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const float l0 = acc[b] + U[j].bias[0], l1 = acc[NB + b] + U[j].bias[1];
                    if (l0 > bv[b]) { bv[b] = l0; bi[b] = v; }
                    if (l1 > bv[b]) { bv[b] = l1; bi[b] = v + 1; }
                    if (a.logits && b < B && lane < 2)
                        a.logits[((size_t)t * B + b) * V + v + lane] = lane == 0 ? l0 : l1;
                }
            }
        }
        if (lane == 0) {
#pragma unroll
            for (int b = 0; b < NB; b++) { s_bv[wid * MAXB + b] = bv[b]; s_bi[wid * MAXB + b] = bi[b]; }
        }
        __syncthreads();
        TRACE_EV(a.L, 2);
        if (tid < B) {
            float v = -INFINITY;
            int i = 0x7fffffff;
            for (int ww = 0; ww < WPB; ww++) {
                const float vv = s_bv[ww * MAXB + tid];
                const int ii = s_bi[ww * MAXB + tid];
                if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
            }
            const size_t pa = a.ex.amax(a.L, t & 1, tid, fi);
            const u4 rec = {as_uint(v), tag, (unsigned)i, tag};      // (value, index) pairs in one store
            __builtin_amdgcn_raw_buffer_store_b128(rec, xa, (unsigned)(pa * 8), 0, CP_SC1);
        }
    };
    auto prefetch_f = [&]() {
        const int nu = V / 2, kr = nrounds(nu, nF);
#pragma unroll
        for (int j = 0; j < PH; j++)
            if (j < kr) load_f(j, min((j * nF + fi) * WPB + wid, nu - 1));
        load_gamma<DC>(gp, rw, a.g_final, lane);
    };
    // this step's fed tokens replace the previous step's argmax
    auto feed_tokens = [&](int t_) {
        for (int b = tid; b < B; b += BLOCK)
            if (t_ < a.n_feed[b]) s_tok[b] = a.feed[(size_t)t_ * B + b];
        __syncthreads();
    };

    if (role == R_AC) {
        // ---------------- A + C ----------------
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            feed_tokens(t);
            for (int l = 0; l < a.L; l++) {
                TRACE_EV(l, 0);
                const LayerOff w = load_layer(a.layers + l);
                // opaque per layer: keeps the compiler from hoisting every
                // phase's lane-dependent addresses out of the loops
                asm volatile("" : "+v"(lane));
                // ---- A: rms_norm -> qkv + bias -> RoPE -> Q / KN / VN.  Unit u =
                // rows (2u, 2u+1), so RoPE pairs stay in one wavefront; Q, KN and
                // VN are adjacent in the exchange row.
                const int nuA = 3 * D / 2;
                auto load_aw = [&](int j, int u) { load_a(j, w, u, 0); };
                if (!pre) {
                    prefetch(nuA, nAC, load_aw);
                    load_gamma<DC>(gp, rw, w.g_attn, lane);
                }
                pre = false;
                if (l == 0) {
                    // embedding rows of this step's tokens (embedding.c:79-84)
                    for (int c = wid; c < nrows * (ldD / 256); c += WPB) {
                        const int r = c / (ldD / 256), col = (c - r * (ldD / 256)) * 256 + 4 * lane;
                        *reinterpret_cast<f4 *>(xs + r * ldD + col) = ld4<0>(rw, (a.embed + (size_t)s_tok[r] * ldD + col) * 4);
                    }
                } else {
                    stage_rows<NB * 6 / WPB + 1>(xs, ldD, D, nrows, a.ex.x2(l - 1, 0), xstride, xa, tag, wid, lane, wt);
                }
                lds_barrier();
                TRACE_EV(l, 1);
                {
                    float rs[NB];
                    rms_lds<NB, DC>(xs, ldD, D, w.eps_attn, lane, rs);
                    auto part_a = [&](int j, float *sj) { part_lds<2, NB, DC, true>(U[j].w, xs, ldD, rs, gp, lane, sj); };
                    auto epi_a = [&](int j, int u, const float *acc, float *out) {
                        const int n = 2 * u;
                        const int sec = n / D;
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            float v0 = acc[b] + U[j].bias[0], v1 = acc[NB + b] + U[j].bias[1];
                            if (sec < 2 && a.rope) {     // rope.c:28-32
                                const float c = bcast(rc[j], b), sn = bcast(rsn[j], b);
                                const float e = v0, o = v1;
                                v0 = e * c - o * sn;
                                v1 = e * sn + o * c;
                            }
                            if (lane == 0) { out[wid * NB * 2 + b * 2] = v0; out[wid * NB * 2 + b * 2 + 1] = v1; }
                        }
                    };
                    gemv(nuA, nAC, 2, load_aw, part_a, epi_a, [&](const float *out, int u0, int nv) {
                        write_block<2, NB, PH * WPB>(out, xa, a.ex.q(l, 0), xstride, u0, min(nuA, u0 + nv), B, tag, lane);
                    }, l, 9);
                }
                TRACE_EV(l, 2);

                // ---- C: out_proj + bias + residual -> X1 (transformer.c:408);
                // its rows load while attention runs
                const int nuC = D / 2;
                auto load_c = [&](int j, int u) {
                    load_u(j, w.wo + 2 * (size_t)u * ldD, w.bo + 2 * (size_t)u, w.bo + 2 * (size_t)u + 1);
                };
                prefetch(nuC, nAC, load_c);
                if (ns == 1)
                    stage_rows<NB * 6 / WPB + 1>(as, ldD, D, nrows, a.ex.att(l, 0), xstride, xa, tag, wid, lane, wt);
                else
                    stage_att_split(as, ldD, B * H, H, ns, a.ex.ao(a.L, l), a.ex.aml(a.L, l), xa, tag, wid, lane, wt);
                lds_barrier();
                TRACE_EV(l, 4);
                gemv(nuC, nAC, 2, load_c, [&](int j, float *sj) {
                    float rs[NB];
                    part_lds<2, NB, DC, false>(U[j].w, as, ldD, rs, gp, lane, sj);
                }, [&](int j, int u, const float *acc, float *out) {
                    if (lane == 0) {
#pragma unroll
                        for (int b = 0; b < NB; b++)
#pragma unroll
                            for (int r = 0; r < 2; r++)
                                out[wid * NB * 2 + b * 2 + r] = xs[b * ldD + 2 * u + r] + (acc[r * NB + b] + U[j].bias[r]);
                    }
                }, [&](const float *out, int u0, int nv) {
                    write_block<2, NB, PH * WPB>(out, xa, a.ex.x1(l, 0), xstride, u0, min(nuC, u0 + nv), B, tag, lane);
                }, l, 11);
                TRACE_EV(l, 5);
                // the next layer's first A rounds (after the last layer: layer 0
                // of the next step, at the next position), loaded while D, E and
                // the lm_head run
                {
                    const bool last = l + 1 == a.L;
                    const LayerOff wn = load_layer(a.layers + (last ? 0 : l + 1));
                    prefetch(nuA, nAC, [&](int j, int u) { load_a(j, wn, u, last ? 1 : 0); });
                    load_gamma<DC>(gp, rw, wn.g_attn, lane);
                    pre = true;
                }
            }
            if (reduce_g(tag)) { t++; break; }
        }
    } else if (role == R_ATT) {
        // ---------------- attention ----------------
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            for (int l = 0; l < a.L; l++) {
                TRACE_EV(l, 0);
                asm volatile("" : "+v"(lane));
                // ---- B: attention.  Record r = (b*H + h)*ns + split runs on
                // attention workgroup r mod n_att; its K/V loads are issued as
                // soon as the previous layer's records are stored.  Split sp
                // takes the 32-key chunks c = sp + ns*(w + 8k) (wavefront w), CPW
                // of them per pass, all loaded before the pass waits for the
                // query.  Scores: lanes 0-31 hold dims 0-31, lanes 32-63 dims 32-63
                // of a chunk's 32 keys (key = j0 + (lane & 31)); P.V: lane = output
                // dim.  One split (ns = 1) writes the head's ATT row; more write
                // (O, m, l) records that phase C merges.
                for (int r = r0; r < B * H * ns; r += nAT) {
                    const int bh = r / ns, sp = r - bh * ns;
                    const int b = bh / H, h = bh - b * H;
                    const int p = s_pos[b], S = p + 1, nch = (S + CH - 1) / CH;
                    const int half = lane >> 5, kl = lane & 31;
                    const size_t head = (((size_t)l * B + b) * H + h) * kv_head;
                    float m_run = -INFINITY, l_run = 0.f, o_run = 0.f;
                    float q = 0.f, kn = 0.f, vn = 0.f;
                    bool have_q = false;
                    float *qe = s_qe + wid * (DK + CPW * CH);
                    for (int c0 = sp + ns * wid; c0 < nch; c0 += CPW * ns * WPB) {
                        // cached keys (positions < p) of the pass's chunks, issued
                        // before the waits (keys >= p masked to 0; they are
                        // never used unmasked)
                        float kt[CPW][32], vr[CPW][CH];
                        int cn = -1;                         // the pass's chunk holding position p
#pragma unroll
                        for (int cc = 0; cc < CPW; cc++) {
                            const int c = c0 + cc * ns * WPB, j0 = c * CH, key = j0 + kl;
                            if (c < nch) {
                                const unsigned kvo = (unsigned)((head + (size_t)(32 * half) * a.max_seq + key) * 4);
                                const unsigned vvo = (unsigned)((head + (size_t)j0 * DK + lane) * 4);
#pragma unroll
                                for (int i = 0; i < 32; i++) {
                                    const float tv = ld1s<CP_SC1>(rk, kvo, (unsigned)(i * a.max_seq * 4));
                                    kt[cc][i] = key < p ? tv : 0.f;
                                }
#pragma unroll
                                for (int jj = 0; jj < CH; jj++) {
                                    const float tv = ld1s<CP_SC1>(rv, vvo, (unsigned)(jj * DK * 4));
                                    vr[cc][jj] = j0 + jj < p ? tv : 0.f;
                                }
                            } else {
#pragma unroll
                                for (int i = 0; i < 32; i++) kt[cc][i] = 0.f;
#pragma unroll
                                for (int jj = 0; jj < CH; jj++) vr[cc][jj] = 0.f;
                            }
                            if (c < nch && p >= j0 && p < j0 + CH) cn = cc;
                        }
                        const bool has_new = cn >= 0;
                        if (!have_q || has_new) {
                            // this step's q (first pass) and new k, v (the pass
                            // holding position p), polled together: one hop
                            const size_t qp = a.ex.q(l, b) + h * DK + lane;
                            const bool wq = !have_q;
                            wt.reset();
                            for (;;) {
                                u2 v0 = {0u, tag}, v1 = {0u, tag}, v2 = {0u, tag};
                                if (wq) v0 = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)(qp * 8), 0, CP_SC1);
                                if (has_new) {
                                    v1 = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)((qp + D) * 8), 0, CP_SC1);
                                    v2 = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)((qp + 2 * D) * 8), 0, CP_SC1);
                                }
                                if (wq) q = as_float(v0.x);
                                kn = as_float(v1.x);
                                vn = as_float(v2.x);
                                if (__all(v0.y == tag && v1.y == tag && v2.y == tag) || !wt.again()) break;
                            }
                            have_q = true;
                            TRACE_EV(l, 9);
                        }
                        asm volatile("" : "+v"(q));     // no hoisting of the per-half q selects below
                        if (has_new) {
                            // append position p to the caches (transformer.c:76-93);
                            // the stores complete (the workgroup barrier's wait)
                            // before the workgroup's later steps
                            st1(rk, (head + (size_t)lane * a.max_seq + p) * 4, kn);    // K^T[d][p]
                            st1(rv, (head + (size_t)p * DK + lane) * 4, vn);           // V[p][d]
                        }
                        // q and the chunks' weights go through this wavefront's QE
                        // slot (16-byte LDS reads that every lane of a half-wave
                        // shares): no per-lane selects between broadcast registers
                        qe[lane] = q;
                        float s[CPW];
                        bool valid[CPW];
#pragma unroll
                        for (int cc = 0; cc < CPW; cc++) {
                            s[cc] = 0.f;
#pragma unroll
                            for (int i = 0; i < 32; i += 4) {
                                const f4 qv = *reinterpret_cast<const f4 *>(qe + 32 * half + i);
                                s[cc] += qv.x * kt[cc][i] + qv.y * kt[cc][i + 1] + qv.z * kt[cc][i + 2] + qv.w * kt[cc][i + 3];
                            }
                        }
#pragma unroll
                        for (int cc = 0; cc < CPW; cc++) {
                            s[cc] += __shfl_xor(s[cc], 32, WAVE);                  // transformer.c:291-297
                            s[cc] = s[cc] * scale;
                            const int key = (c0 + cc * ns * WPB) * CH + kl;
                            valid[cc] = c0 + cc * ns * WPB < nch && key < S;
                        }
                        if (has_new) {
                            const float sn = wave_sum(q * kn) * scale;
#pragma unroll
                            for (int cc = 0; cc < CPW; cc++)
                                if ((c0 + cc * ns * WPB) * CH + kl == p) s[cc] = sn;
                        }
                        float mx = -INFINITY;
#pragma unroll
                        for (int cc = 0; cc < CPW; cc++) mx = fmaxf(mx, valid[cc] ? s[cc] : -INFINITY);
                        const float m_new = fmaxf(m_run, wave_max(mx));
                        const float fa = expf(m_run - m_new);
                        float e[CPW], es = 0.f;
#pragma unroll
                        for (int cc = 0; cc < CPW; cc++) {
                            e[cc] = valid[cc] ? expf(s[cc] - m_new) : 0.f;
                            es += e[cc];
                            if (lane < CH) qe[DK + cc * CH + lane] = e[cc];
                        }
                        float o = 0.f;
#pragma unroll
                        for (int cc = 0; cc < CPW; cc++) {
#pragma unroll
                            for (int jj = 0; jj < CH; jj += 4) {
                                const f4 ev = *reinterpret_cast<const f4 *>(qe + DK + cc * CH + jj);
                                o += ev.x * vr[cc][jj] + ev.y * vr[cc][jj + 1] + ev.z * vr[cc][jj + 2] + ev.w * vr[cc][jj + 3];
                            }
                        }
                        if (has_new) {
                            float ep = 0.f;
#pragma unroll
                            for (int cc = 0; cc < CPW; cc++)
                                if (cc == cn) ep = bcast(e[cc], p - (c0 + cc * ns * WPB) * CH);
                            o += ep * vn;
                        }
                        l_run = l_run * fa + wave_sum(half ? 0.f : es);
                        o_run = o_run * fa + o;
                        m_run = m_new;
                    }
                    // a split whose first wavefront has no chunk still waits for this
                    // step's query, so its record is never written ahead of the step
                    if (!have_q && wid == 0) (void)poll1(xa, (long)(a.ex.q(l, b) + h * DK + lane), tag, wt);
                    s_part[wid * (DK + 2) + lane] = o_run;
                    if (lane == 0) { s_part[wid * (DK + 2) + DK] = m_run; s_part[wid * (DK + 2) + DK + 1] = l_run; }
                    TRACE_EV(l, 10);
                    lds_barrier();          // the cache appends complete at the record's closing barrier
                    TRACE_EV(l, 11);
                    if (wid == 0) {
                        // lanes w < WPB: wavefront w's weight e^(m_w - M)
                        const float mw = lane < WPB ? s_part[lane * (DK + 2) + DK] : -INFINITY;
                        const float M = wave_max(mw);
                        const float fw = mw == -INFINITY ? 0.f : expf(mw - M);
                        float O = 0.f, Ls = 0.f;
#pragma unroll
                        for (int ww = 0; ww < WPB; ww++) {
                            const float f = bcast(fw, ww);
                            O += s_part[ww * (DK + 2) + lane] * f;
                            Ls += s_part[ww * (DK + 2) + DK + 1] * f;
                        }
                        if (ns == 1) {
                            put(xa, a.ex.att(l, b) + h * DK + lane, O / Ls, tag);
                        } else {
                            put(xa, a.ex.ao(a.L, l) + (size_t)r * DK + lane, O, tag);
                            if (lane < 2) put(xa, a.ex.aml(a.L, l) + (size_t)r * 2 + lane, lane == 0 ? M : Ls, tag);
                        }
                    }
                    __syncthreads();
                }
                TRACE_EV(l, 3);
            }
            if (reduce_g(tag)) { t++; break; }
        }
    } else if (role == R_D) {
        // ---------------- D (+ lm_head) ----------------
        // rms_norm(X1) -> gate/up + bias -> SwiGLU -> ACT (nn.c:61-78,
        // simd.h:394-397); unit f = gate row f and up row f
        auto load_d = [&](const LayerOff &w_, int j, int f) {
            load_u(j, w_.wgu + 2 * (size_t)f * ldD, w_.bg + (size_t)f, w_.bu + (size_t)f);
        };
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            for (int l = 0; l < a.L; l++) {
                TRACE_EV(l, 0);
                const LayerOff w = load_layer(a.layers + l);
                asm volatile("" : "+v"(lane));
                auto load_dw = [&](int j, int f) { load_d(w, j, f); };
                if (l == 0 && !pre) {
                    prefetch(F, nDD, load_dw);
                    load_gamma<DC>(gp, rw, w.g_ffn, lane);
                }
                pre = false;
                stage_rows<NB * 6 / WPB + 1>(x1s, ldD, D, nrows, a.ex.x1(l, 0), xstride, xa, tag, wid, lane, wt);
                lds_barrier();
                TRACE_EV(l, 6);
                float rs[NB];
                rms_lds<NB, DC>(x1s, ldD, D, w.eps_ffn, lane, rs);
                TRACE_EV(l, 12);
                gemv(F, nDD, 1, load_dw, [&](int j, float *sj) {
                    part_lds<2, NB, DC, true>(U[j].w, x1s, ldD, rs, gp, lane, sj);
                }, [&](int j, int f, const float *acc, float *out) {
                    if (lane == 0) {
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            const float gg = acc[b] + U[j].bias[0], up = acc[NB + b] + U[j].bias[1];
                            out[wid * NB + b] = (gg / (1.0f + expf(-gg))) * up;
                        }
                    }
                }, [&](const float *out, int u0, int nv) {
                    write_block<1, NB, PH * WPB>(out, xa, a.ex.act(l, 0), xstride, u0, min(F, u0 + nv), B, tag, lane);
                }, l, 14);
                TRACE_EV(l, 7);
                if (l + 1 < a.L) {
                    const LayerOff wn = load_layer(a.layers + l + 1);
                    prefetch(F, nDD, [&](int j, int f) { load_d(wn, j, f); });
                    load_gamma<DC>(gp, rw, wn.g_ffn, lane);
                } else {
                    prefetch_f();
                }
            }
            lm_head(tag);
            {
                // layer 0 of the next step, loaded while the partials are gathered
                const LayerOff w0 = load_layer(a.layers);
                prefetch(F, nDD, [&](int j, int f) { load_d(w0, j, f); });
                load_gamma<DC>(gp, rw, w0.g_ffn, lane);
                pre = true;
            }
            if (reduce_g(tag)) { t++; break; }
        }
    } else {
        // ---------------- E (+ lm_head) ----------------
        // down + bias + residual -> X2 (transformer.c:415); unit n = row n,
        // PE rounds held in registers
        typename WPiece<BF>::T wr[PE][FCMAX];
        float bdn[PE];
        const int FC = ldF / 256;
        auto load_e = [&](const LayerOff &w_, int j, int n) {
#pragma unroll
            for (int c = 0; c < FCMAX; c++)
                if (c < FC) wr[j][c] = ld_piece<BF>(rm, w_.wd + (size_t)n * ldF + c * 256, lane);
            bdn[j] = ld1<0>(rw, (w_.bd + (size_t)n) * 4);
        };
        auto prefetch_e = [&](const LayerOff &w_) {
            const int kr = nrounds(D, nEE);
#pragma unroll
            for (int j = 0; j < PE; j++)
                if (j < kr) load_e(w_, j, min(unit(j, kr), D - 1));
        };
        bool pre_e = false;                 // layer 0's rows held
        constexpr bool EF_EARLY = NB <= 2;
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            if (EF_EARLY && a.L == 1) prefetch_f();
            for (int l = 0; l < a.L; l++) {
                TRACE_EV(l, 0);
                const LayerOff w = load_layer(a.layers + l);
                asm volatile("" : "+v"(lane));
                if (l == 0 && !pre_e) prefetch_e(w);
                pre_e = false;
                stage_rows<NB * 6 / WPB + 1>(x1s, ldD, D, nrows, a.ex.x1(l, 0), xstride, xa, tag, wid, lane, wt);
                stage_rows<NB * 16 / WPB + 1>(acts, ldF, F, nrows, a.ex.act(l, 0), xstride, xa, tag, wid, lane, wt);
                lds_barrier();
                TRACE_EV(l, 8);
                const int kr = nrounds(D, nEE);
                for (int k0 = 0; k0 < kr; k0 += PE) {
                    if (k0 > 0) {
#pragma unroll
                        for (int j = 0; j < PE; j++)
                            if (k0 + j < kr) load_e(w, j, min(unit(k0 + j, kr), D - 1));
                    }
#pragma unroll
                    for (int j = 0; j < PE; j++) {
                        const int n = unit(k0 + j, kr);
                        if (k0 + j >= kr || n >= D) continue;
                        float *out = s_out + j * (WPB * NB);
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            float sum = 0.f;
#pragma unroll
                            for (int c = 0; c < FCMAX; c++) {
                                if (c >= FC) continue;
                                const f4 y = *reinterpret_cast<const f4 *>(acts + b * ldF + c * 256 + 4 * lane);
                                const f4 wv = widen(wr[j][c]);
                                sum += wv.x * y.x + wv.y * y.y + wv.z * y.z + wv.w * y.w;
                            }
                            sum = wave_sum(sum);
                            if (lane == 0) out[wid * NB + b] = x1s[b * ldD + n] + (sum + bdn[j]);
                        }
                    }
                    TRACE_EV(l, 14);
                    lds_barrier();
                    TRACE_EV(l, 15);
                    if (wid == 0) {
                        const int u0 = (r0 * kr + k0) * WPB;
                        write_block<1, NB, PE * WPB>(s_out, xa, a.ex.x2(l, 0), xstride, u0,
                                                     min(D, u0 + min(PE, kr - k0) * WPB), B, tag, lane);
                    }
                    lds_barrier();
                }
                TRACE_EV(l, 13);
                if (l + 1 < a.L) prefetch_e(load_layer(a.layers + l + 1));
                // the lm_head rounds ride along through the last layer (in
                // registers beside its rows, where both fit)
                if (EF_EARLY ? l + 2 == a.L : l + 1 == a.L) prefetch_f();
            }
            lm_head(tag);
            prefetch_e(load_layer(a.layers));   // layer 0 of the next step
            pre_e = true;
            if (reduce_g(tag)) { t++; break; }
        }
    }
    if (g0 == 0 && tid < B) a.pos[tid] = s_pos[tid];
    if (g0 == 0 && tid == 0) *a.steps_done = t;
}


template <int NB, int DC, bool BF>
__global__ void __launch_bounds__(BLOCK)
decode_v3(DecodeArgs a) {
    decode_v3_body<NB, DC, BF>(a, gridDim.x, blockIdx.x);
}

}  // namespace dnnhip
