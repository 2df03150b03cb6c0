// decode_kernel.hip -- the persistent gfx950 decode kernel.
//
// One launch runs n_steps of the GPT token loop of masc-it/dnn.c
// (decoder_lm_generate, gpt.c:306-375) for B <= 8 rows at once:
//
//   per layer (transformer_block_forward_cached_ex, transformer.c:211-416)
//     A  rms_norm(x) -> qkv GEMV + bias -> RoPE(q, k) -> Q / KN / VN
//     B  attention of one (row, head) per workgroup: each wavefront takes
//        32-key chunks of the S = pos+1 keys with a running max / sum, the
//        workgroup merges the wavefronts' (o, max, sum) in LDS; the wavefront
//        holding position pos appends the new K/V row to the caches
//     C  out_proj GEMV + bias + residual                      -> X1
//     D  rms_norm(X1) -> gate/up GEMV + bias -> SwiGLU        -> ACT
//     E  down GEMV + bias + residual                          -> X2
//   then
//     F  rms_norm(X2) -> tied lm_head GEMV + bias -> argmax partial per workgroup
//     G  every workgroup reduces the partials (first index of the maximum,
//        gpt.c:220-230) and feeds the token to the next step's embedding rows
//
// Synchronisation is dataflow, not grid barriers.  Every value a wavefront
// produces for other workgroups is one 8-byte (value, tag) store with
// device-coherent (sc1) caching; the tag is the global step id.  A workgroup
// that needs a row (the input of a GEMV phase) stages it into LDS once: its 8
// wavefronts split the row, poll their parts until every value carries this
// step's tag, write it to LDS, and meet at a workgroup barrier.  Each
// dependency costs one coherent hop, no L2 writeback/invalidate is issued, and
// the row crosses the fabric once per workgroup rather than once per wavefront.
// A wavefront issues the weight loads of its work unit before the staging
// poll, so weight streaming overlaps the wait.
//
// Weights are out-major (row n = the K inputs of output n, padded to a multiple
// of 256 floats): each output is one contiguous, coalesced dot product owned by
// one wavefront; unit u of a phase goes to wavefront u mod (8 * grid), counted
// workgroup-fastest, so consecutive units land on different CUs.  Every global
// access goes through a buffer descriptor sized to its tensor, so the hardware
// range-checks it (out-of-range loads read 0, stores are dropped).

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
template <int NB, int DC>
__device__ __forceinline__ void decode_v3_body(const DecodeArgs &a, const int G, const int g0) {
    extern __shared__ float smem[];
    int *s_tok = reinterpret_cast<int *>(smem);                 // [MAXB]
    int *s_pos = s_tok + MAXB;                                  // [MAXB]
    int *s_done = s_pos + MAXB;                                 // [MAXB]
    float *s_bv = reinterpret_cast<float *>(s_done + MAXB);     // [WPB][MAXB]
    int *s_bi = reinterpret_cast<int *>(s_bv + WPB * MAXB);     // [WPB][MAXB]
    float *s_part = reinterpret_cast<float *>(s_bi + WPB * MAXB);   // [WPB][DK + 2]
    float *s_out = s_part + WPB * (DK + 2);                     // [2][WPB][2 * MAXB]
    float *s_qe = s_out + 2 * WPB * 2 * MAXB;                   // [WPB][DK + CH]
    const int ldD = a.ldD, ldF = a.ldF;
    float *xs = smem + (LDS_HEAD_WORDS + 3) / 4 * 4;            // [NB][ldD] layer input (raw)
    float *as = xs + NB * ldD;                                  // [NB][ldD] attention output
    float *x1s = as + NB * ldD;                                 // [NB][ldD] X1 (raw)
    float *acts = x1s + NB * ldD;                               // [NB][ldF] SwiGLU output

    const int tid = threadIdx.x;
    int lane = tid & (WAVE - 1);
    const int wid = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int gw = wid * G + g0;                                // workgroup-fastest wave numbering
    const int nw = G * WPB;
    const int B = a.B, D = a.D, H = a.H, F = a.F, V = a.V;
    const int nrows = B < NB ? B : NB;
    const int ns = a.ex.ns > 1 ? a.ex.ns : 1;                  // workgroups per (row, head)
    Waiter wt{a.err};

    const size_t kv_head = (size_t)DK * a.max_seq;              // floats per (layer, row, head)
    const rsrc_t rw = buf(a.wts, a.wts_bytes);
    const rsrc_t xa = buf(a.xa, a.ex.total(a.L) * 8);
    const size_t kv_bytes = ((size_t)a.L * B * H * kv_head + (size_t)CH * DK) * 4;   // incl. the padding
    const rsrc_t rk = buf(a.kc, kv_bytes);
    const rsrc_t rv = buf(a.vc, kv_bytes);
    const size_t sin_off = (size_t)a.rope_rows * (DK / 2) * 4;      // bytes
    const rsrc_t rrope = buf(a.rope, a.rope ? 2 * sin_off : 0);
    const size_t xstride = a.ex.per_row();
    const float scale = 1.0f / sqrtf((float)DK);

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
    for (; t < a.n_steps; t++) {
        const unsigned tag = a.step0 + (unsigned)t;
        for (int b = tid; b < B; b += BLOCK)
            if (t < a.n_feed[b]) s_tok[b] = a.feed[(size_t)t * B + b];
        __syncthreads();

        for (int l = 0; l < a.L; l++) {
            TRACE_EV(l, 0);
            const LayerOff w = load_layer(a.layers + l);
            // opaque per layer: keeps the compiler from hoisting every phase's
            // lane-dependent addresses out of the loops (they would all stay
            // live for the whole launch and spill)
            asm volatile("" : "+v"(lane));

            // ---- A: rms_norm -> qkv + bias -> RoPE -> Q / KN / VN.  Unit u = rows
            // (2u, 2u+1) (RoPE pairs stay in one wavefront); the units of round k
            // of workgroup g are (k*G + g)*WPB + wid, so a workgroup's outputs are
            // contiguous (Q, KN and VN are adjacent in the exchange row).
            {
                constexpr int UP = 2;                // rounds preloaded before the wait
                const int nu = 3 * D / 2;
                RowUnit<2, DC> U[UP];
                float rc[UP], rsn[UP];               // lane b < NB: cos / sin of row b's position
                f4 g[DC];
                auto load_a = [&](int k, int u) {
                    const int n = 2 * u;
                    const size_t bo[2] = {w.bqkv + (size_t)n, w.bqkv + (size_t)n + 1};
                    load_unit<2, DC>(U[k], rw, w.wqkv + (size_t)n * ldD, ldD, bo, lane);
                    const int sec = n / D, j = (n - sec * D) % DK;
                    rc[k] = 1.f; rsn[k] = 0.f;
                    if (sec < 2 && a.rope && lane < NB) {
                        const size_t ti = ((size_t)s_pos[lane < B ? lane : B - 1] * (DK / 2) + j / 2) * 4;
                        rc[k] = ld1<0>(rrope, ti);
                        rsn[k] = ld1<0>(rrope, sin_off + ti);
                    }
                };
                auto comp_a = [&](int k, int u, const float (&rs)[NB], float *out) {
                    const int n = 2 * u;
                    float acc[2][NB];
                    dot_lds<2, NB, DC, true>(U[k].w, xs, ldD, rs, g, lane, acc);
                    const int sec = n / D;
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        float v0 = acc[0][b] + U[k].bias[0], v1 = acc[1][b] + U[k].bias[1];
                        if (sec < 2 && a.rope) {     // rope.c:28-32
                            const float c = bcast(rc[k], b), sn = bcast(rsn[k], b);
                            const float e = v0, o = v1;
                            v0 = e * c - o * sn;
                            v1 = e * sn + o * c;
                        }
                        if (lane == 0) { out[wid * NB * 2 + b * 2] = v0; out[wid * NB * 2 + b * 2 + 1] = v1; }
                    }
                };
#pragma unroll
                for (int k = 0; k < UP; k++)
                    if ((k * G + g0) * WPB + wid < nu) load_a(k, (k * G + g0) * WPB + wid);
                const bool busy = g0 * WPB < nu;
                if (busy) load_gamma<DC>(g, rw, w.g_attn, lane);
                if (l == 0) {
                    // embedding rows of this step's tokens (embedding.c:79-84)
                    for (int c = wid; c < nrows * (ldD / 256); c += WPB) {
                        const int r = c / (ldD / 256), col = (c - r * (ldD / 256)) * 256 + 4 * lane;
                        *reinterpret_cast<f4 *>(xs + r * ldD + col) = ld4<0>(rw, (a.embed + (size_t)s_tok[r] * ldD + col) * 4);
                    }
                } else if (busy) {
                    stage_rows<NB * 6 / WPB + 1>(xs, ldD, D, nrows, a.ex.x2(l - 1, 0), xstride, xa, tag, wid, lane, wt);
                }
                __syncthreads();
                TRACE_EV(l, 1);
                if (busy) {
                    float rs[NB];
                    rms_lds<NB, DC>(xs, ldD, D, w.eps_attn, lane, rs);
                    for (int k = 0; (k * G + g0) * WPB < nu; k++) {
                        const int u0 = (k * G + g0) * WPB, u = u0 + wid;
                        float *out = s_out + (k & 1) * (WPB * 2 * MAXB);
                        if (u < nu) {
                            if (k >= UP) load_a(0, u);
                            comp_a(k < UP ? k : 0, u, rs, out);
                        }
                        __syncthreads();
                        if (wid == 0) write_block<2, NB>(out, xa, a.ex.q(l, 0), xstride, u0, nu, B, tag, lane);
                    }
                }
            }

            TRACE_EV(l, 2);
            // ---- B: attention.  Record r = (b*H + h)*ns + split runs on workgroup
            // G-1-(r mod G): the last workgroups, which hold no phase-A units for
            // the model shapes served, so their K/V loads start as the layer
            // starts.  Split sp takes the 32-key chunks c = sp + ns*(w + 8k)
            // (wavefront w).  Scores: lanes 0-31 hold dims 0-31, lanes 32-63 dims
            // 32-63 of the chunk's 32 keys (key = j0 + (lane & 31)); P.V: lane =
            // output dim.  One split (ns = 1) writes the head's ATT row; more
            // write (O, m, l) records that phase C merges.
            for (int r = G - 1 - g0; r < B * H * ns; r += G) {
                const int bh = r / ns, sp = r - bh * ns;
                const int b = bh / H, h = bh - b * H;
                const int p = s_pos[b], S = p + 1, nch = (S + CH - 1) / CH;
                const int half = lane >> 5, kl = lane & 31;
                const size_t head = (((size_t)l * B + b) * H + h) * kv_head;
                float m_run = -INFINITY, l_run = 0.f, o_run = 0.f;
                float q = 0.f, kn = 0.f, vn = 0.f;
                bool have_q = false;
                for (int c = sp + ns * wid; c < nch; c += ns * WPB) {
                    const int j0 = c * CH, key = j0 + kl;
                    // cached keys (positions < p) of this chunk, issued before the waits
                    // (unconditional loads, then a select: keys >= p hold stale or
                    // neighbouring values, all finite, never used unmasked)
                    float kt[32], vr[CH];
                    const unsigned kvo = (unsigned)((head + (size_t)(32 * half) * a.max_seq + key) * 4);
                    const unsigned vvo = (unsigned)((head + (size_t)j0 * DK + lane) * 4);
#pragma unroll
                    for (int i = 0; i < 32; i++) {
                        const float tv = ld1s<CP_SC1>(rk, kvo, (unsigned)(i * a.max_seq * 4));
                        kt[i] = key < p ? tv : 0.f;
                    }
#pragma unroll
                    for (int jj = 0; jj < CH; jj++) {
                        const float tv = ld1s<CP_SC1>(rv, vvo, (unsigned)(jj * DK * 4));
                        vr[jj] = j0 + jj < p ? tv : 0.f;
                    }
                    const bool has_new = p >= j0 && p < j0 + CH;
                    if (!have_q || has_new) {
                        // this step's q (first chunk) and new k, v (the chunk
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
                        // append position p to the caches (transformer.c:76-93); the
                        // stores are waited for (device scope) before the workgroup
                        // leaves the head, so they complete before any later step
                        // reads position p
                        st1(rk, (head + (size_t)lane * a.max_seq + p) * 4, kn);    // K^T[d][p]
                        st1(rv, (head + (size_t)p * DK + lane) * 4, vn);           // V[p][d]
                    }
                    // q and the chunk's weights go through this wavefront's QE slot
                    // (16-byte LDS reads that every lane of a half-wave shares):
                    // no per-lane selects between broadcast registers
                    float *qe = s_qe + wid * (DK + CH);
                    qe[lane] = q;
                    float s = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; i += 4) {
                        const f4 qv = *reinterpret_cast<const f4 *>(qe + 32 * half + i);
                        s += qv.x * kt[i] + qv.y * kt[i + 1] + qv.z * kt[i + 2] + qv.w * kt[i + 3];
                    }
                    s += __shfl_xor(s, 32, WAVE);                              // transformer.c:291-297
                    s = s * scale;
                    if (has_new) {
                        const float sn = wave_sum(q * kn) * scale;
                        if (key == p) s = sn;
                    }
                    const bool valid = key < S;
                    const float m_c = wave_max(valid ? s : -INFINITY);
                    const float m_new = fmaxf(m_run, m_c);
                    const float e = valid ? expf(s - m_new) : 0.f;
                    const float fa = expf(m_run - m_new);
                    if (lane < CH) qe[DK + lane] = e;
                    float o = 0.f;
#pragma unroll
                    for (int jj = 0; jj < CH; jj += 4) {
                        const f4 ev = *reinterpret_cast<const f4 *>(qe + DK + jj);
                        o += ev.x * vr[jj] + ev.y * vr[jj + 1] + ev.z * vr[jj + 2] + ev.w * vr[jj + 3];
                    }
                    if (has_new) o += bcast(e, p - j0) * vn;
                    l_run = l_run * fa + wave_sum(half ? 0.f : e);
                    o_run = o_run * fa + o;
                    m_run = m_new;
                }
                // a split whose first wavefront has no chunk still waits for this
                // step's query, so its record is never written ahead of the step
                if (!have_q && wid == 0) (void)poll1(xa, (long)(a.ex.q(l, b) + h * DK + lane), tag, wt);
                s_part[wid * (DK + 2) + lane] = o_run;
                if (lane == 0) { s_part[wid * (DK + 2) + DK] = m_run; s_part[wid * (DK + 2) + DK + 1] = l_run; }
                TRACE_EV(l, 10);
                __syncthreads();
                TRACE_EV(l, 11);
                if (wid == 0) {
                    float M = -INFINITY;
                    for (int ww = 0; ww < WPB; ww++) M = fmaxf(M, s_part[ww * (DK + 2) + DK]);
                    float O = 0.f, Ls = 0.f;
                    for (int ww = 0; ww < WPB; ww++) {
                        const float mw = s_part[ww * (DK + 2) + DK];
                        const float f = mw == -INFINITY ? 0.f : expf(mw - M);
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
                __builtin_amdgcn_s_waitcnt(0x0f70);                           // vmcnt(0): cache appends done
                __syncthreads();
            }

            TRACE_EV(l, 3);
            // ---- C: out_proj + bias + residual -> X1 (transformer.c:408); unit u =
            // rows (2u, 2u+1), workgroup-contiguous rounds as in A
            {
                constexpr int UP = 2;
                const int nu = D / 2;
                RowUnit<2, DC> U[UP];
                f4 g[DC];
                float rs[NB];
                auto load_c = [&](int k, int u) {
                    const size_t bo[2] = {w.bo + 2 * (size_t)u, w.bo + 2 * (size_t)u + 1};
                    load_unit<2, DC>(U[k], rw, w.wo + 2 * (size_t)u * ldD, ldD, bo, lane);
                };
                auto comp_c = [&](int k, int u, float *out) {
                    float acc[2][NB];
                    dot_lds<2, NB, DC, false>(U[k].w, as, ldD, rs, g, lane, acc);
                    if (lane == 0) {
#pragma unroll
                        for (int b = 0; b < NB; b++)
#pragma unroll
                            for (int r = 0; r < 2; r++)
                                out[wid * NB * 2 + b * 2 + r] = xs[b * ldD + 2 * u + r] + (acc[r][b] + U[k].bias[r]);
                    }
                };
#pragma unroll
                for (int k = 0; k < UP; k++)
                    if ((k * G + g0) * WPB + wid < nu) load_c(k, (k * G + g0) * WPB + wid);
                const bool busy = g0 * WPB < nu;
                if (busy) {
                    if (ns == 1)
                        stage_rows<NB * 6 / WPB + 1>(as, ldD, D, nrows, a.ex.att(l, 0), xstride, xa, tag, wid, lane, wt);
                    else
                        stage_att_split(as, ldD, B * H, H, ns, a.ex.ao(a.L, l), a.ex.aml(a.L, l), xa, tag, wid, lane, wt);
                }
                __syncthreads();
                TRACE_EV(l, 4);
                if (busy) {
                    for (int k = 0; (k * G + g0) * WPB < nu; k++) {
                        const int u0 = (k * G + g0) * WPB, u = u0 + wid;
                        float *out = s_out + (k & 1) * (WPB * 2 * MAXB);
                        if (u < nu) {
                            if (k >= UP) load_c(0, u);
                            comp_c(k < UP ? k : 0, u, out);
                        }
                        __syncthreads();
                        if (wid == 0) write_block<2, NB>(out, xa, a.ex.x1(l, 0), xstride, u0, nu, B, tag, lane);
                    }
                }
            }

            TRACE_EV(l, 5);
            // ---- D: rms_norm(X1) -> gate/up + bias -> SwiGLU -> ACT  (nn.c:61-78,
            // simd.h:394-397); unit f = gate row f and up row f
            {
                constexpr int UP = 2;
                const int nu = F;
                RowUnit<2, DC> U[UP];
                f4 g[DC];
                auto load_d = [&](int k, int f) {
                    const size_t bo[2] = {w.bg + (size_t)f, w.bu + (size_t)f};
                    load_unit<2, DC>(U[k], rw, w.wgu + 2 * (size_t)f * ldD, ldD, bo, lane);
                };
                auto comp_d = [&](int k, const float (&rs)[NB], float *out) {
                    float acc[2][NB];
                    dot_lds<2, NB, DC, true>(U[k].w, x1s, ldD, rs, g, lane, acc);
                    if (lane == 0) {
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            const float gg = acc[0][b] + U[k].bias[0], up = acc[1][b] + U[k].bias[1];
                            out[wid * NB + b] = (gg / (1.0f + expf(-gg))) * up;
                        }
                    }
                };
#pragma unroll
                for (int k = 0; k < UP; k++)
                    if ((k * G + g0) * WPB + wid < nu) load_d(k, (k * G + g0) * WPB + wid);
                const bool busy = g0 * WPB < nu;
                if (busy) load_gamma<DC>(g, rw, w.g_ffn, lane);
                if (busy || g0 * WPB < D)            // phase E reads X1S for its residual
                    stage_rows<NB * 6 / WPB + 1>(x1s, ldD, D, nrows, a.ex.x1(l, 0), xstride, xa, tag, wid, lane, wt);
                __syncthreads();
                TRACE_EV(l, 6);
                if (busy) {
                    float rs[NB];
                    rms_lds<NB, DC>(x1s, ldD, D, w.eps_ffn, lane, rs);
                    for (int k = 0; (k * G + g0) * WPB < nu; k++) {
                        const int u0 = (k * G + g0) * WPB, u = u0 + wid;
                        float *out = s_out + (k & 1) * (WPB * 2 * MAXB);
                        if (u < nu) {
                            if (k >= UP) load_d(0, u);
                            comp_d(k < UP ? k : 0, rs, out);
                        }
                        __syncthreads();
                        if (wid == 0) write_block<1, NB>(out, xa, a.ex.act(l, 0), xstride, u0, nu, B, tag, lane);
                    }
                }
            }

            TRACE_EV(l, 7);
            // ---- E: down + bias + residual -> X2 (transformer.c:415); unit n = row n
            {
                const int nu = D, FC = ldF / 256;
                f4 wr[FCMAX];
                float bdn = 0.f;
                auto load_down = [&](int n) {
#pragma unroll
                    for (int k = 0; k < FCMAX; k++)
                        if (k < FC) wr[k] = ld4<CP_NT>(rw, (w.wd + (size_t)n * ldF + k * 256 + 4 * lane) * 4);
                    bdn = ld1<0>(rw, (w.bd + (size_t)n) * 4);
                };
                if (g0 * WPB + wid < nu) load_down(g0 * WPB + wid);
                const bool busy = g0 * WPB < nu;
                if (busy)
                    stage_rows<NB * 16 / WPB + 1>(acts, ldF, F, nrows, a.ex.act(l, 0), xstride, xa, tag, wid, lane, wt);
                __syncthreads();
                TRACE_EV(l, 8);
                if (busy) {
                    for (int k = 0; (k * G + g0) * WPB < nu; k++) {
                        const int u0 = (k * G + g0) * WPB, n = u0 + wid;
                        float *out = s_out + (k & 1) * (WPB * 2 * MAXB);
                        if (n < nu) {
                            if (k >= 1) load_down(n);
#pragma unroll
                            for (int b = 0; b < NB; b++) {
                                float sum = 0.f;
#pragma unroll
                                for (int c = 0; c < FCMAX; c++) {
                                    if (c >= FC) continue;
                                    const f4 y = *reinterpret_cast<const f4 *>(acts + b * ldF + c * 256 + 4 * lane);
                                    sum += wr[c].x * y.x + wr[c].y * y.y + wr[c].z * y.z + wr[c].w * y.w;
                                }
                                sum = wave_sum(sum);
                                if (lane == 0) out[wid * NB + b] = x1s[b * ldD + n] + (sum + bdn);
                            }
                        }
                        __syncthreads();
                        if (wid == 0) write_block<1, NB>(out, xa, a.ex.x2(l, 0), xstride, u0, nu, B, tag, lane);
                    }
                }
            }
        }

        TRACE_EV(a.L, 0);
        // ---- F: final rms_norm -> tied lm_head + bias -> per-workgroup argmax
        asm volatile("" : "+v"(lane));
        {
            constexpr int UP = 1;
            float bv[NB];
            int bi[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
            const int nu = V / 2;
            RowUnit<2, DC> U[UP];
            f4 g[DC];
            auto load_f = [&](int k, int u) {
                const int v = 2 * u;
                const size_t bo[2] = {a.lm_bias + (size_t)v, a.lm_bias + (size_t)v + 1};
                load_unit<2, DC>(U[k], rw, a.embed + (size_t)v * ldD, ldD, bo, lane);
            };
            auto comp_f = [&](int k, int u, const float (&rs)[NB]) {
                const int v = 2 * u;
                float acc[2][NB];
                dot_lds<2, NB, DC, true>(U[k].w, xs, ldD, rs, g, lane, acc);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const float l0 = acc[0][b] + U[k].bias[0], l1 = acc[1][b] + U[k].bias[1];
                    if (l0 > bv[b]) { bv[b] = l0; bi[b] = v; }
                    if (l1 > bv[b]) { bv[b] = l1; bi[b] = v + 1; }
                    if (a.logits && b < B && lane < 2)
                        a.logits[((size_t)t * B + b) * V + v + lane] = lane == 0 ? l0 : l1;
                }
            };
            if (gw < nu) load_gamma<DC>(g, rw, a.g_final, lane);
            if (g0 < nu)
                stage_rows<NB * 6 / WPB + 1>(xs, ldD, D, nrows, a.ex.x2(a.L - 1, 0), xstride, xa, tag, wid, lane, wt);
            __syncthreads();
            TRACE_EV(a.L, 1);
            if (gw < nu) {
                // the rows are loaded after the wait, one unit at a time: more
                // rows in registers, or rows held across the polling loop, are
                // spilled here, one load at a time
                float rs[NB];
                rms_lds<NB, DC>(xs, ldD, D, a.eps_final, lane, rs);
                for (int u = gw; u < nu; u += nw) {
                    load_f(0, u);
                    comp_f(0, u, rs);
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
                const size_t pa = a.ex.amax(a.L, t & 1, tid, g0);
                put(xa, pa, v, tag);
                put(xa, pa + 1, __builtin_bit_cast(float, i), tag);
            }
        }

        // ---- G: every workgroup reduces the partials -> next token (same in all);
        // wavefront w reduces rows w, w + 8, ...
        for (int b = wid; b < B; b += WPB) {
            float v = -INFINITY;
            int i = 0x7fffffff;
            // every workgroup's partial in one polling pass (4 per lane)
            for (int gb = 0; gb < G; gb += 4 * WAVE) {
                u4 q[4];
                wt.reset();
                for (;;) {
                    bool ok = true;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int gg = gb + k * WAVE + lane;
                        const size_t pa = a.ex.amax(a.L, t & 1, b, gg < G ? gg : 0);
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
                    if (gg < G && (vv > v || (vv == v && ii < i))) { v = vv; i = ii; }
                }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float vv = __shfl_xor(v, o, WAVE);
                const int ii = __shfl_xor(i, o, WAVE);
                if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
            }
            if (lane == 0) {
                if (i < 0 || i >= V) i = 0;     // all-NaN row: argmax keeps index 0
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
            if (all) { t++; break; }
        }
    }
    if (g0 == 0 && tid < B) a.pos[tid] = s_pos[tid];
    if (g0 == 0 && tid == 0) *a.steps_done = t;
}

template <int NB, int DC>
__global__ void __launch_bounds__(BLOCK)
decode_v3(DecodeArgs a) {
    decode_v3_body<NB, DC>(a, gridDim.x, blockIdx.x);
}

#define DNNHIP_INST(NB, DC) template __global__ void decode_v3<NB, DC>(DecodeArgs);
DNNHIP_INST(1, 1) DNNHIP_INST(1, 2) DNNHIP_INST(1, 3)
DNNHIP_INST(2, 1) DNNHIP_INST(2, 2) DNNHIP_INST(2, 3)
DNNHIP_INST(4, 1) DNNHIP_INST(4, 2) DNNHIP_INST(4, 3)
DNNHIP_INST(8, 1) DNNHIP_INST(8, 2) DNNHIP_INST(8, 3)

#ifdef DNNHIP_TRACE
extern "C" int dnn_hip_trace_arm(int step) {
    static unsigned long long zero[256 * TRACE_L * TRACE_E];
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_trace), zero, sizeof zero) != hipSuccess) return -1;
    return hipMemcpyToSymbol(HIP_SYMBOL(g_trace_step), &step, sizeof step) == hipSuccess ? 0 : -1;
}
extern "C" int dnn_hip_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_trace), sizeof(unsigned long long) * 256 * TRACE_L * TRACE_E) ==
                   hipSuccess ? 0 : -1;
}
#endif

const void *decode_kernel_for(int nb, int dc) {
#define DNNHIP_PICK(NB, DC) if (nb == NB && dc == DC) return reinterpret_cast<const void *>(&decode_v3<NB, DC>);
    DNNHIP_PICK(1, 1) DNNHIP_PICK(1, 2) DNNHIP_PICK(1, 3)
    DNNHIP_PICK(2, 1) DNNHIP_PICK(2, 2) DNNHIP_PICK(2, 3)
    DNNHIP_PICK(4, 1) DNNHIP_PICK(4, 2) DNNHIP_PICK(4, 3)
    DNNHIP_PICK(8, 1) DNNHIP_PICK(8, 2) DNNHIP_PICK(8, 3)
    return nullptr;
}

}  // namespace dnnhip
