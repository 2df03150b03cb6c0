// decode_stream.hip -- the streaming gfx950 decode kernel for one or two rows.
//
// Same token loop and arithmetic as decode_v3 (gpt.c:306-375,
// transformer.c:211-416), scheduled so that no weight byte is fetched on the
// critical path:
//
//   * GEMV workgroups (0 .. NG-1) own a balanced, contiguous share of every
//     GEMV phase (QKV, out_proj, gate/up, down, lm_head).  Wavefront 0 streams
//     the workgroup's weight rows, in the order they will be consumed and
//     about one layer ahead, into one LDS ring with direct-to-LDS DMA
//     (buffer_load ... lds); it issues nothing else, so the in-order
//     completion of vector memory lets it wait for exactly the phase the
//     workgroup needs next (s_waitcnt vmcnt(n)).  Wavefront 7, the stager,
//     issues every poll of the exchange arena, so a poll never queues behind a
//     weight fetch; it stages the phase input into LDS (with the RMSNorm
//     applied where the phase has one).  All eight meet at a workgroup barrier,
//     wavefronts 1-6 compute the phase's dot products from the ring, and after
//     a second barrier the stager writes the workgroup's outputs as one
//     coalesced block of tagged pairs.
//   * attention workgroups (the last B*H*NS): NS per (row, head); split s takes
//     the 32-key chunks c = s (mod NS), wavefront w the chunks with
//     c / NS = w (mod 8).  The cached keys and values of a chunk are loaded
//     into registers before the query is polled.  A split writes its
//     unnormalised partial (o, m, l); the out_proj stagers merge the NS
//     partials of each head as they stage the attention row.
//
// Synchronisation between workgroups is the tagged-pair dataflow of decode_v3
// (decode_kernel.hip): a value is this step's when its tag is the step id.

#include "decode_device.h"

namespace dnnhip {

namespace {

constexpr int NPH = 5;              // phase kinds: A (qkv), C (out), D (gate/up), E (down), F (lm_head)
enum { K_A = 0, K_C = 1, K_D = 2, K_E = 3, K_F = 4 };

// LDS head (ints): tok[8] pos[8] done[8] misc[8], the phase table
// ph[kind][8] = {nu, R, chunks, u0, n, -, -, -} (units of the phase, rows per
// unit, 256-float chunks per row, this workgroup's first unit and unit count),
// then PST / PEND [S_NBIAS] of the weight stream.
enum { H_TOK = 0, H_POS = 8, H_DONE = 16, H_STOP = 24, H_PH = 32, H_PST = 72, H_PEND = 72 + S_NBIAS };
enum { P_NU = 0, P_R = 1, P_CH = 2, P_U0 = 3, P_N = 4 };

__device__ __forceinline__ int ufl(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) void *)p;
}

// One direct-to-LDS DMA: 64 lanes x 16 bytes from rsrc + voff (per lane) to
// LDS [m0 + 16 * lane].  Non-temporal: weights are read once per step.  M0 is
// written here only; nothing else in these kernels uses it.
__device__ __forceinline__ void dma16(rsrc_t r, unsigned lds, unsigned voff, unsigned soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
// 64 lanes x 4 bytes (a gather: voff per lane) to LDS [m0 + 4 * lane].
__device__ __forceinline__ void dma4(rsrc_t r, unsigned lds, unsigned voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(lds), "v"(voff), "s"(r) : "memory", "m0");
}

// Wait until at most n vector memory operations of this wavefront are
// outstanding (n wave-uniform).  The counter holds at most 63, so n >= 63
// waits for nothing.
#define W1(k) case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
#define W8(k) W1(k) W1(k + 1) W1(k + 2) W1(k + 3) W1(k + 4) W1(k + 5) W1(k + 6) W1(k + 7)
__device__ __forceinline__ void wait_vm(int n) {
    n = ufl(n);
    switch (n) {
        W8(0) W8(8) W8(16) W8(24) W8(32) W8(40) W8(48)
        W1(56) W1(57) W1(58) W1(59) W1(60) W1(61) W1(62)
        default: break;
    }
}
#undef W8
#undef W1

__device__ __forceinline__ void raw_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);     // lgkmcnt(0): this wavefront's LDS traffic is done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ LayerOff lds_layer(const LayerOff *lt, int l) {
    LayerOff w = lt[l];
    w.wqkv = ufl(w.wqkv); w.bqkv = ufl(w.bqkv); w.wo = ufl(w.wo); w.bo = ufl(w.bo);
    w.g_attn = ufl(w.g_attn); w.g_ffn = ufl(w.g_ffn); w.wgu = ufl(w.wgu); w.bg = ufl(w.bg);
    w.bu = ufl(w.bu); w.wd = ufl(w.wd); w.bd = ufl(w.bd);
    return w;
}

// ---------------------------------------------------------------------------
// The workgroup's weight stream (wavefront 0).  Stream order per step: for
// each layer the workgroup's units of A, C, D, E, then of F.  Each phase
// starts with one bias item (a 64-lane dword gather of the phase's biases into
// a bias slot; gate/up: gate biases in lanes 0-31, up in 32-63), then one item
// per unit: R rows x ch chunks of 256 floats, one ring slot per chunk, units
// in order.  A phase is admitted when fewer than S_NBIAS phases are in flight;
// a unit when the ring has room for it.
struct Issuer {
    int rs;
    unsigned ring, bias;            // LDS byte addresses of the ring / bias slots
    unsigned vl;                    // 16 * lane: the per-lane byte offset of a slot DMA
    int it, il, ik, ij;             // next item: step, layer, kind, unit (-1: bias item)
    int n, R, ch;                   // the current phase: units, rows per unit, chunks per row
    uint32_t row;                   // byte offset of the next unit's first row
    uint32_t ld;                    // byte distance of a unit's rows
    int slot;                       // tail % rs
    int tail, head;                 // ring slots issued / released
    int btail, bhead;               // phases issued / released
    int issued;                     // DMA instructions issued
};

struct PhaseOf {                    // this workgroup's units of one phase
    int R, ch, u0, n;
};

__device__ __forceinline__ PhaseOf phase_of(const int *ph, int k) {
    PhaseOf p;
    const int *e = ph + 8 * k;
    p.R = ufl(e[P_R]); p.ch = ufl(e[P_CH]); p.u0 = ufl(e[P_U0]); p.n = ufl(e[P_N]);
    return p;
}

// Issue up to `budget` DMA instructions of the stream, as far as they fit.
// s_pst / s_pend [S_NBIAS]: ring slot where each phase in flight starts, and
// the issue count after its last DMA.
__device__ __forceinline__ void top_up(Issuer &q, int budget, const DecodeArgs &a, const LayerOff *lt, const int *ph,
                                       int *s_pst, int *s_pend, rsrc_t rw, int lane) {
    while (q.it < a.n_steps && budget > 0) {
        if (q.ij < 0) {
            // phase start: its parameters, then the bias gather
            if (q.btail - q.bhead >= S_NBIAS) return;
            const PhaseOf p = phase_of(ph, q.ik);
            q.n = p.n; q.R = p.R; q.ch = p.ch;
            const LayerOff *w = lt + (q.ik == K_F ? 0 : q.il);
            uint32_t rbase, ld, bbase;
            int i = lane;
            switch (q.ik) {
                case K_A: rbase = w->wqkv + 2u * p.u0 * a.ldD; ld = a.ldD; bbase = w->bqkv + 2u * p.u0;
                          if (i >= 2 * p.n) i = 0; break;
                case K_C: rbase = w->wo + (uint32_t)p.u0 * a.ldD; ld = a.ldD; bbase = w->bo + p.u0;
                          if (i >= p.n) i = 0; break;
                case K_D: rbase = w->wgu + 2u * p.u0 * a.ldD; ld = a.ldD;
                          if ((i & 31) >= p.n) i = 0;
                          bbase = (i < 32 ? w->bg : w->bu - 32u) + p.u0; break;
                case K_E: rbase = w->wd + (uint32_t)p.u0 * a.ldF; ld = a.ldF; bbase = w->bd + p.u0;
                          if (i >= p.n) i = 0; break;
                default:  rbase = a.embed + (uint32_t)p.u0 * a.ldD; ld = a.ldD; bbase = a.lm_bias + p.u0;
                          if (i >= p.n) i = 0; break;
            }
            q.row = (uint32_t)ufl((int)rbase) * 4u;
            q.ld = (uint32_t)ufl((int)ld) * 4u;
            dma4(rw, q.bias + (unsigned)((q.btail % S_NBIAS) * S_BSLOT), (bbase + (uint32_t)i) * 4u);
            if (lane == 0) s_pst[q.btail % S_NBIAS] = q.slot;
            q.issued++;
            budget--;
            q.ij = 0;
        } else {
            const int slots = q.R * q.ch;
            if (q.tail + slots - q.head > q.rs) return;
            for (int r = 0; r < q.R; r++)
                for (int c = 0; c < q.ch; c++) {
                    dma16(rw, q.ring + (unsigned)(q.slot * S_SLOT), q.vl, q.row + (uint32_t)r * q.ld + (uint32_t)c * 1024u);
                    q.slot = q.slot + 1 == q.rs ? 0 : q.slot + 1;
                }
            q.row += (uint32_t)q.R * q.ld;
            q.tail += slots;
            q.issued += slots;
            budget -= slots;
            q.ij++;
        }
        if (q.ij == q.n) {                      // phase complete (possibly empty): record it, go to the next
            if (lane == 0) s_pend[q.btail % S_NBIAS] = q.issued;
            q.btail++;
            q.ij = -1;
            if (q.ik == K_F) { q.ik = K_A; q.il = 0; q.it++; }
            else if (q.ik == K_E) { if (q.il == a.L - 1) q.ik = K_F; else { q.ik = K_A; q.il++; } }
            else q.ik++;
        }
    }
}

// ---------------------------------------------------------------------------
// stager helpers

// Poll NQ chunks of 128 tagged values (64 lanes x 2 pairs) of nrows rows of n
// values (row r at pair index base0 + r * stride), chunks c_begin ..
// c_begin+NQ-1 of the rows' concatenation (past the end: the last chunk
// again), until every value inside the rows carries tag.
template <int NQ>
__device__ __forceinline__ void poll_rows(u4 (&q)[NQ], rsrc_t xa, size_t base0, size_t stride, int n, int nrows,
                                          int c_begin, unsigned tag, int lane, Waiter &wt) {
    const int cpr = (n + 127) / 128, total = nrows * cpr;
    wt.reset();
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int c = min(c_begin + i, total - 1);
            const int r = c / cpr, col = (c - r * cpr) * 128 + 2 * lane;
            q[i] = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)((base0 + r * stride + col) * 8), 0, CP_SC1);
            const unsigned t0 = q[i].y, t1 = q[i].w;
            ok &= (col >= n || t0 == tag) && (col + 1 >= n || t1 == tag);
        }
        if (__all(ok) || !wt.again()) break;
    }
}

// Stage NB rows of n <= 128*NCH values into xs (raw) and, if norm, ys =
// (x * rs) * gamma with rs = 1/sqrtf(sum(x^2) / n + eps) (norm.c:433-471).
// The values are either polled (row b at pair index base + b * stride) or,
// when emb is set, embedding rows of the tokens tok[b].
template <int NB, int NCH>
__device__ __forceinline__ void stage_in(float *xs, float *ys, int ld, int n, bool norm, float eps, uint32_t g_off,
                                         bool emb, const int *tok, uint32_t embed, rsrc_t rw, rsrc_t xa, size_t base,
                                         size_t stride, unsigned tag, int lane, Waiter &wt) {
    u2 g[NCH];
    if (norm) {
#pragma unroll
        for (int c = 0; c < NCH; c++)
            g[c] = __builtin_amdgcn_raw_buffer_load_b64(rw, (g_off + (unsigned)(c * 128 + 2 * lane)) * 4u, 0, 0);
    }
    float x[NB][NCH][2];
    if (emb) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t row = embed + (uint32_t)tok[b] * (uint32_t)ld;
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                const u2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, (row + (unsigned)(c * 128 + 2 * lane)) * 4u, 0, 0);
                x[b][c][0] = as_float(v.x);
                x[b][c][1] = as_float(v.y);
            }
        }
    } else {
        u4 q[NB * NCH];
        poll_rows<NB * NCH>(q, xa, base, stride, n, NB, 0, tag, lane, wt);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                x[b][c][0] = as_float(q[b * NCH + c].x);
                x[b][c][1] = as_float(q[b * NCH + c].z);
            }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int col = c * 128 + 2 * lane;
            if (col < n) {
                xs[b * ld + col] = x[b][c][0];
                ss += x[b][c][0] * x[b][c][0];
            }
            if (col + 1 < n) {
                xs[b * ld + col + 1] = x[b][c][1];
                ss += x[b][c][1] * x[b][c][1];
            }
        }
        if (norm) {
            const float rs = 1.0f / sqrtf(wave_sum(ss) * (1.0f / (float)n) + eps);
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                const int col = c * 128 + 2 * lane;
                if (col < n) ys[b * ld + col] = (x[b][c][0] * rs) * as_float(g[c].x);
                if (col + 1 < n) ys[b * ld + col + 1] = (x[b][c][1] * rs) * as_float(g[c].y);
            }
        }
    }
}

// Stage the attention rows: merge the NS split partials of each (row, head)
// (transformer.c:349-397 computes the same softmax-weighted sum in one pass).
// Record r = (b*H + h)*NS + s; AO chunk c holds records 2c (lanes 0-31) and
// 2c+1 (lanes 32-63), two dims per lane; the AML chunk holds (m, l) of record
// lane.  att = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, M = max_s m_s.
template <int NS>
__device__ __forceinline__ void stage_att(float *as, int ld, int nrec, int H, size_t ao, size_t aml, rsrc_t xa,
                                          unsigned tag, int lane, Waiter &wt) {
    constexpr int NQ = S_MAXREC / 2;          // AO chunks
    constexpr int CPH = NS / 2;               // AO chunks per head
    const int nco = nrec / 2;
    u4 q[NQ + 1];
    wt.reset();
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int c = min(i, nco - 1);
            q[i] = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)((ao + (size_t)c * 128 + 2 * lane) * 8), 0, CP_SC1);
            ok &= q[i].y == tag && q[i].w == tag;
        }
        const int r = min(lane, nrec - 1);
        q[NQ] = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)((aml + (size_t)r * 2) * 8), 0, CP_SC1);
        ok &= q[NQ].y == tag && q[NQ].w == tag;
        if (__all(ok) || !wt.again()) break;
    }
    const float m = lane < nrec ? as_float(q[NQ].x) : -INFINITY;
    const float lsum = lane < nrec ? as_float(q[NQ].z) : 0.f;
    float M = m;
    M = fmaxf(M, dpp<0xb1, 0xf>(M, -INFINITY));                 // groups of 2 lanes
    if (NS == 4) M = fmaxf(M, dpp<0x4e, 0xf>(M, -INFINITY));    // groups of 4 lanes
    const float wgt = m == -INFINITY ? 0.f : expf(m - M);
    float den = wgt * lsum;
    den += dpp<0xb1, 0xf>(den, 0.f);
    if (NS == 4) den += dpp<0x4e, 0xf>(den, 0.f);
    const int half = lane >> 5;
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int c = 0; c < NQ; c++) {
        const float wl = bcast(wgt, (2 * c) & 63), wh = bcast(wgt, (2 * c + 1) & 63);
        const float ww = half ? wh : wl;
        o0 += ww * as_float(q[c].x);
        o1 += ww * as_float(q[c].z);
        if (c % CPH == CPH - 1) {
            const int hb = c / CPH;
            if (hb * NS < nrec) {
                o0 += __shfl_xor(o0, 32, WAVE);
                o1 += __shfl_xor(o1, 32, WAVE);
                const float d = bcast(den, (hb * NS) & 63);
                if (lane < 32) {
                    const int b = hb / H, h = hb - b * H;
                    as[b * ld + h * DK + 2 * lane] = o0 / d;
                    as[b * ld + h * DK + 2 * lane + 1] = o1 / d;
                }
            }
            o0 = 0.f;
            o1 = 0.f;
        }
    }
}

// Lm_head argmax partials of every GEMV workgroup -> the token of each row
// (first index of the maximum, gpt.c:220-230).  Returns row b's token in
// lane-uniform form through tok[b].
template <int NB>
__device__ __forceinline__ void reduce_amax(int (&tok)[NB], const Exch5 &ex, int L, int par, int NG, int V,
                                            rsrc_t xa, unsigned tag, int lane, Waiter &wt) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float v = -INFINITY;
        int i = 0x7fffffff;
        for (int gb = 0; gb < NG; gb += WAVE) {
            const int gg = gb + lane;
            const size_t pa = ex.amax(L, par, b, gg < NG ? gg : NG - 1);
            u4 q;
            wt.reset();
            for (;;) {
                q = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)(pa * 8), 0, CP_SC1);
                if (__all(q.y == tag && q.w == tag) || !wt.again()) break;
            }
            const float vv = as_float(q.x);
            const int ii = (int)q.z;
            if (gg < NG && (vv > v || (vv == v && ii < i))) { v = vv; i = ii; }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float vv = __shfl_xor(v, o, WAVE);
            const int ii = __shfl_xor(i, o, WAVE);
            if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
        }
        i = ufl(i);
        if (i < 0 || i >= V) i = 0;              // all-NaN row: argmax keeps index 0
        tok[b] = i;
    }
}

}  // namespace

template <int NB, int DC>
__global__ void __launch_bounds__(BLOCK)
decode_v5(StreamArgs sa) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const DecodeArgs &a = sa.a;
    const Exch5 &ex = sa.ex;
    const Lds5 &lo = sa.lds;
    int *hd = reinterpret_cast<int *>(lds);
    int *s_ph = hd + H_PH;
    float *s_rope = reinterpret_cast<float *>(lds + lo.rope);
    LayerOff *s_lt = reinterpret_cast<LayerOff *>(lds + lo.lt);
    float *s_part = reinterpret_cast<float *>(lds + lo.part);
    float *s_best = reinterpret_cast<float *>(lds + lo.best);
    float *s_out = reinterpret_cast<float *>(lds + lo.out);
    float *xs = reinterpret_cast<float *>(lds + lo.xs);
    float *ys = reinterpret_cast<float *>(lds + lo.ys);
    float *as = reinterpret_cast<float *>(lds + lo.as);
    float *x1s = reinterpret_cast<float *>(lds + lo.x1s);
    float *acts = reinterpret_cast<float *>(lds + lo.acts);

    const int tid = threadIdx.x;
    int lane = tid & (WAVE - 1);
    const int wid = ufl(tid / WAVE);
    const int g0 = blockIdx.x, NG = sa.ng;
    const int B = a.B, D = a.D, H = a.H, F = a.F, V = a.V, L = a.L;
    const int ldD = a.ldD, ldF = a.ldF;
    constexpr int NS = NB == 1 ? 4 : 2;
    Waiter wt{a.err};
    const rsrc_t rw = buf(a.wts, a.wts_bytes);
    const rsrc_t xa = buf(a.xa, ex.total(L) * 8);

    // ---- setup: positions, layer table, phase table, zeroed rows
    for (int i = tid; i < 32; i += BLOCK) hd[i] = (i >= H_POS && i < H_POS + NB) ? a.pos[i - H_POS] : 0;
    for (int i = tid; i < L * (int)(sizeof(LayerOff) / 4); i += BLOCK)
        reinterpret_cast<uint32_t *>(s_lt)[i] = reinterpret_cast<const uint32_t *>(a.layers)[i];
    for (int i = tid; i < NB * (2 * ldD + (2 * ldD > ldF ? 2 * ldD : ldF)); i += BLOCK)
        xs[i] = 0.f;                                         // XS, X1S, YS / AS / ACTS are adjacent
    if (tid < NPH) {
        const int k = tid;
        const int nu = k == K_A ? 3 * D / 2 : k == K_C ? D : k == K_D ? F : k == K_E ? D : V;
        const int R = (k == K_A || k == K_D) ? 2 : 1;
        const int ch = k == K_E ? ldF / 256 : ldD / 256;
        const int u0 = (int)((long)nu * g0 / NG), u1 = (int)((long)nu * (g0 + 1) / NG);
        int *e = s_ph + 8 * k;
        e[P_NU] = nu; e[P_R] = R; e[P_CH] = ch; e[P_U0] = u0; e[P_N] = u1 - u0;
    }
    __syncthreads();

    if (g0 >= NG) {
        // ================= attention workgroup =================
        const int ai = g0 - NG;
        const int b = ai / (H * NS), h = (ai / NS) % H, sp = ai % NS;
        const size_t kv_head = (size_t)DK * a.max_seq;
        const size_t kv_bytes = ((size_t)L * B * H * kv_head + (size_t)CH * DK) * 4;
        const rsrc_t rk = buf(a.kc, kv_bytes);
        const rsrc_t rv = buf(a.vc, kv_bytes);
        const float scale = 1.0f / sqrtf((float)DK);
        const int half = lane >> 5, kl = lane & 31;
        int t = 0;
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            const int p = hd[H_POS + b] + t, S = p + 1, nch = (S + CH - 1) / CH;
            for (int l = 0; l < L; l++) {
                const size_t head = (((size_t)l * B + b) * H + h) * kv_head;
                float m_run = -INFINITY, l_run = 0.f, o_run = 0.f;
                float q = 0.f;
                bool have_q = false;
                for (int c = sp + NS * wid; c < nch; c += NS * WPB) {
                    const int j0 = c * CH, key = j0 + kl;
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
                    float kn = 0.f, vn = 0.f;
                    {
                        // this step's q (first chunk) and new k, v (the chunk holding
                        // position p), polled together
                        const size_t qp = ex.qkv(l, b) + h * DK + lane;
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
                    }
                    asm volatile("" : "+v"(q));
                    if (has_new) {
                        // append position p (transformer.c:76-93); the stores are
                        // waited for at the end of the layer (later steps read them)
                        st1(rk, (head + (size_t)lane * a.max_seq + p) * 4, kn);
                        st1(rv, (head + (size_t)p * DK + lane) * 4, vn);
                    }
                    float s = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; i++) s += (half ? bcast(q, 32 + i) : bcast(q, i)) * kt[i];
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
                    float o = 0.f;
#pragma unroll
                    for (int jj = 0; jj < CH; jj++) o += bcast(e, jj) * vr[jj];
                    if (has_new) o += bcast(e, p - j0) * vn;
                    l_run = l_run * fa + wave_sum(half ? 0.f : e);
                    o_run = o_run * fa + o;
                    m_run = m_new;
                }
                // a split with no chunk still waits for this step's query, so its
                // record is never written ahead of the step
                if (!have_q && wid == 0) (void)poll1(xa, (long)(ex.qkv(l, b) + h * DK + lane), tag, wt);
                s_part[wid * (DK + 2) + lane] = o_run;
                if (lane == 0) { s_part[wid * (DK + 2) + DK] = m_run; s_part[wid * (DK + 2) + DK + 1] = l_run; }
                __syncthreads();
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
                    const int rec = (b * H + h) * NS + sp;
                    put(xa, ex.ao(l) + (size_t)rec * DK + lane, O, tag);
                    if (lane < 2) put(xa, ex.aml(l) + (size_t)rec * 2 + lane, lane == 0 ? M : Ls, tag);
                }
                __builtin_amdgcn_s_waitcnt(0x0f70);                           // vmcnt(0): cache appends done
                __syncthreads();
            }
            if (a.eos >= 0) {
                // the stop rule of the GEMV workgroups, from the same partials
                if (wid == 0) {
                    int tok[NB];
                    reduce_amax<NB>(tok, ex, L, t & 1, NG, V, xa, tag, lane, wt);
                    if (lane == 0) {
                        int all = 1;
#pragma unroll
                        for (int bb = 0; bb < NB; bb++) {
                            if (t >= a.n_feed[bb] - 1 && tok[bb] == a.eos) hd[H_DONE + bb] = 1;
                            all &= hd[H_DONE + bb];
                        }
                        hd[H_STOP] = all;
                    }
                }
                __syncthreads();
                if (hd[H_STOP]) break;
            }
        }
        return;
    }

    if (wid == WPB - 1) {
        // ================= stager =================
        int tok[NB];
        int t = 0;
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (t < a.n_feed[b]) hd[H_TOK + b] = a.feed[(size_t)t * B + b];
                tok[b] = ufl(hd[H_TOK + b]);
            }
            if (a.rope) {
                const rsrc_t rr = buf(a.rope, (size_t)a.rope_rows * DK * 4);
                const size_t sin_off = (size_t)a.rope_rows * (DK / 2);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const size_t pp = (size_t)(hd[H_POS + b] + t) * (DK / 2);
                    s_rope[b * 64 + lane] = ld1<0>(rr, (lane < 32 ? pp + lane : sin_off + pp + lane - 32) * 4);
                }
            }
            for (int l = 0; l < L; l++) {
                const LayerOff w = lds_layer(s_lt, l);
                // ---- A input: layer input -> XS, normalised -> YS
                stage_in<NB, 2 * DC>(xs, ys, ldD, D, true, s_lt[l].eps_attn, w.g_attn, l == 0, tok, a.embed, rw, xa,
                                     l == 0 ? 0 : ex.x2(l - 1, 0), ex.x2(0, 1) - ex.x2(0, 0), tag, lane, wt);
                raw_barrier();                                   // B1
                raw_barrier();                                   // B2: outputs in OUT
                {
                    const float *out = s_out + (size_t)((4 * l + K_A) & 1) * lo.sout;
                    const int *e = s_ph + 8 * K_A;
                    const int n2 = 2 * e[P_N], u0 = e[P_U0];
                    for (int i = lane; i < NB * n2; i += WAVE) {
                        const int b = i / n2, j = i - b * n2;
                        put(xa, ex.qkv(l, b) + 2 * (size_t)u0 + j, out[i], tag);
                    }
                }
                // ---- C input: attention rows -> AS
                stage_att<NS>(as, ldD, (int)ex.nrec(), H, ex.ao(l), ex.aml(l), xa, tag, lane, wt);
                raw_barrier();
                raw_barrier();
                {
                    const float *out = s_out + (size_t)((4 * l + K_C) & 1) * lo.sout;
                    const int *e = s_ph + 8 * K_C;
                    const int n = e[P_N], u0 = e[P_U0];
                    for (int i = lane; i < NB * n; i += WAVE) {
                        const int b = i / n, j = i - b * n;
                        put(xa, ex.x1(l, b) + (size_t)u0 + j, out[i], tag);
                    }
                }
                // ---- D input: X1 -> X1S, normalised -> YS
                stage_in<NB, 2 * DC>(x1s, ys, ldD, D, true, s_lt[l].eps_ffn, w.g_ffn, false, tok, 0, rw, xa,
                                     ex.x1(l, 0), ex.x1(0, 1) - ex.x1(0, 0), tag, lane, wt);
                raw_barrier();
                raw_barrier();
                {
                    const float *out = s_out + (size_t)((4 * l + K_D) & 1) * lo.sout;
                    const int *e = s_ph + 8 * K_D;
                    const int n = e[P_N], u0 = e[P_U0];
                    for (int i = lane; i < NB * n; i += WAVE) {
                        const int b = i / n, j = i - b * n;
                        put(xa, ex.act(l, b) + (size_t)u0 + j, out[i], tag);
                    }
                }
                // ---- E input: ACT -> ACTS
                {
                    constexpr int NQ = 2 * FCMAX;
                    const int cpr = (F + 127) / 128;
                    for (int c0 = 0; c0 < NB * cpr; c0 += NQ) {
                        u4 q[NQ];
                        poll_rows<NQ>(q, xa, ex.act(l, 0), ex.act(0, 1) - ex.act(0, 0), F, NB, c0, tag, lane, wt);
#pragma unroll
                        for (int i = 0; i < NQ; i++) {
                            const int c = c0 + i;
                            if (c < NB * cpr) {
                                const int r = c / cpr, col = (c - r * cpr) * 128 + 2 * lane;
                                if (col < F) acts[r * ldF + col] = as_float(q[i].x);
                                if (col + 1 < F) acts[r * ldF + col + 1] = as_float(q[i].z);
                            }
                        }
                    }
                }
                raw_barrier();
                raw_barrier();
                {
                    const float *out = s_out + (size_t)((4 * l + K_E) & 1) * lo.sout;
                    const int *e = s_ph + 8 * K_E;
                    const int n = e[P_N], u0 = e[P_U0];
                    for (int i = lane; i < NB * n; i += WAVE) {
                        const int b = i / n, j = i - b * n;
                        put(xa, ex.x2(l, b) + (size_t)u0 + j, out[i], tag);
                    }
                }
            }
            // ---- F input: X2 of the last layer, normalised -> YS
            stage_in<NB, 2 * DC>(xs, ys, ldD, D, true, a.eps_final, a.g_final, false, tok, 0, rw, xa, ex.x2(L - 1, 0),
                                 ex.x2(0, 1) - ex.x2(0, 0), tag, lane, wt);
            raw_barrier();
            raw_barrier();                                       // per-wavefront bests in BEST
            if (lane < NB) {
                float v = -INFINITY;
                int i = 0x7fffffff;
                for (int ww = 0; ww < S_NCW; ww++) {
                    const float vv = s_best[(ww * MAXB + lane) * 2];
                    const int ii = __builtin_bit_cast(int, s_best[(ww * MAXB + lane) * 2 + 1]);
                    if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
                }
                const size_t pa = ex.amax(L, t & 1, lane, g0);
                u4 wv = {as_uint(v), tag, (unsigned)i, tag};
                __builtin_amdgcn_raw_buffer_store_b128(wv, xa, (unsigned)(pa * 8), 0, CP_SC1);
            }
            // ---- G: every workgroup's partials -> next token
            int nt[NB];
            reduce_amax<NB>(nt, ex, L, t & 1, NG, V, xa, tag, lane, wt);
            if (lane == 0) {
                int all = 1;
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    hd[H_TOK + b] = nt[b];
                    if (a.eos >= 0 && t >= a.n_feed[b] - 1 && nt[b] == a.eos) hd[H_DONE + b] = 1;
                    all &= hd[H_DONE + b];
                    if (g0 == 0) a.ids[(size_t)t * B + b] = nt[b];
                }
                hd[H_STOP] = a.eos >= 0 && all;
            }
            raw_barrier();                                       // B3: stop flag
            if (hd[H_STOP]) { t++; break; }
        }
        if (g0 == 0 && lane < NB) a.pos[lane] = hd[H_POS + lane] + t;
        if (g0 == 0 && lane == 0) *a.steps_done = t;
        return;
    }

    int *s_pst = hd + H_PST, *s_pend = hd + H_PEND;
    const float *ring = reinterpret_cast<const float *>(lds + lo.ring);
    const float *bslot = reinterpret_cast<const float *>(lds + lo.bias);
    if (wid == 0) {
        // ================= weight stream =================
        Issuer q;
        q.rs = lo.rs;
        q.ring = lds_addr(lds + lo.ring);
        q.bias = lds_addr(lds + lo.bias);
        q.vl = 16u * (unsigned)lane;
        q.it = 0; q.il = 0; q.ik = K_A; q.ij = -1;
        q.n = q.R = q.ch = 0; q.row = q.ld = 0;
        q.slot = q.tail = q.head = q.btail = q.bhead = q.issued = 0;
        top_up(q, 1 << 20, a, s_lt, s_ph, s_pst, s_pend, rw, lane);     // fill the ring
        int t = 0;
        for (; t < a.n_steps; t++) {
            for (int l = 0; l <= L; l++) {
                for (int k = (l == L ? K_F : K_A); k <= (l == L ? K_F : K_E); k++) {
                    asm volatile("" : "+v"(lane));
                    // stream in bounded batches in every window between barriers,
                    // so the weight stream never holds up a barrier for long
                    top_up(q, 24, a, s_lt, s_ph, s_pst, s_pend, rw, lane);
                    // every earlier phase is released, so this one fits; make sure
                    // it is issued, then wait for its last DMA
                    for (int guard = 0; q.btail <= q.bhead && guard < 64; guard++)
                        top_up(q, 64, a, s_lt, s_ph, s_pst, s_pend, rw, lane);
                    if (q.btail > q.bhead) wait_vm(q.issued - ufl(s_pend[q.bhead % S_NBIAS]));
                    else atomicOr(a.err, 2);            // cannot happen: the ring holds any one phase
                    raw_barrier();                      // B1
                    top_up(q, 12, a, s_lt, s_ph, s_pst, s_pend, rw, lane);
                    raw_barrier();                      // B2: the phase's slots are free again
                    const PhaseOf p = phase_of(s_ph, k);
                    q.head += p.n * p.R * p.ch;
                    q.bhead++;
                }
            }
            top_up(q, 24, a, s_lt, s_ph, s_pst, s_pend, rw, lane);
            raw_barrier();                              // B3
            if (hd[H_STOP]) { t++; break; }
        }
        // no LDS DMA may be in flight when the workgroup's LDS is released
        __builtin_amdgcn_s_waitcnt(0x0f70);
        return;
    }

    // ================= compute wavefronts 1 .. S_NCW =================
    const int cw = wid - 1;
    const int FC = ldF / 256;
    int bhead = 0;
    int t = 0;
    for (; t < a.n_steps; t++) {
        for (int l = 0; l <= L; l++) {
            for (int k = (l == L ? K_F : K_A); k <= (l == L ? K_F : K_E); k++) {
                asm volatile("" : "+v"(lane));
                const PhaseOf p = phase_of(s_ph, k);
                raw_barrier();                                   // B1: phase input staged, weights in the ring
                const int ps = ufl(s_pst[bhead % S_NBIAS]);      // the phase's first ring slot
                const float *bs = bslot + (bhead % S_NBIAS) * (S_BSLOT / 4);
                float *out = s_out + (size_t)((4 * l + k) & 1) * lo.sout;
                const int slots = p.R * p.ch;
                if (k == K_E) {
                    f4 y[NB][FCMAX];
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int c = 0; c < FCMAX; c++)
                            if (c < FC) y[b][c] = *reinterpret_cast<const f4 *>(acts + b * ldF + c * 256 + 4 * lane);
                    int hs = ps + cw * slots;
                    hs = hs >= lo.rs ? hs - lo.rs : hs;
                    for (int j = cw; j < p.n; j += S_NCW) {
                        f4 wv[FCMAX];
#pragma unroll
                        for (int c = 0; c < FCMAX; c++) {
                            int sl = hs + c;
                            sl = sl >= lo.rs ? sl - lo.rs : sl;
                            if (c < FC) wv[c] = *reinterpret_cast<const f4 *>(ring + sl * (S_SLOT / 4) + 4 * lane);
                        }
                        const int n = p.u0 + j;
                        const float bd = bs[j];
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            float sum = 0.f;
#pragma unroll
                            for (int c = 0; c < FCMAX; c++) {
                                if (c >= FC) continue;
                                sum += wv[c].x * y[b][c].x + wv[c].y * y[b][c].y + wv[c].z * y[b][c].z + wv[c].w * y[b][c].w;
                            }
                            sum = wave_sum(sum);
                            if (lane == 0) out[b * p.n + j] = x1s[b * ldD + n] + (sum + bd);   // transformer.c:415
                        }
                        hs += S_NCW * slots;
                        while (hs >= lo.rs) hs -= lo.rs;
                    }
                } else {
                    const float *src = k == K_C ? as : ys;
                    f4 y[NB][DC];
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int c = 0; c < DC; c++) y[b][c] = *reinterpret_cast<const f4 *>(src + b * ldD + c * 256 + 4 * lane);
                    float bv[NB];
                    int bi[NB];
#pragma unroll
                    for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
                    int hs = ps + cw * slots;
                    hs = hs >= lo.rs ? hs - lo.rs : hs;
                    for (int j = cw; j < p.n; j += S_NCW) {
                        const int u = p.u0 + j;
                        f4 wv[2][DC];
#pragma unroll
                        for (int r = 0; r < 2; r++)
#pragma unroll
                            for (int c = 0; c < DC; c++) {
                                if (r >= p.R) continue;
                                int sl = hs + r * DC + c;
                                sl = sl >= lo.rs ? sl - lo.rs : sl;
                                wv[r][c] = *reinterpret_cast<const f4 *>(ring + sl * (S_SLOT / 4) + 4 * lane);
                            }
                        float acc[2][NB];
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            float s0 = 0.f, s1 = 0.f;
#pragma unroll
                            for (int c = 0; c < DC; c++) {
                                const f4 yy = y[b][c];
                                s0 += wv[0][c].x * yy.x + wv[0][c].y * yy.y + wv[0][c].z * yy.z + wv[0][c].w * yy.w;
                                if (p.R == 2)
                                    s1 += wv[1][c].x * yy.x + wv[1][c].y * yy.y + wv[1][c].z * yy.z + wv[1][c].w * yy.w;
                            }
                            if (p.R == 2) wave_sum2(s0, s1);
                            else s0 = wave_sum(s0);
                            acc[0][b] = s0;
                            acc[1][b] = s1;
                        }
                        if (k == K_A) {
                            const float b0 = bs[2 * j], b1 = bs[2 * j + 1];
                            const int n = 2 * u, sec = n / D, jj = (n - sec * D) % DK;
#pragma unroll
                            for (int b = 0; b < NB; b++) {
                                float v0 = acc[0][b] + b0, v1 = acc[1][b] + b1;
                                if (sec < 2 && a.rope) {             // rope.c:28-32
                                    const float c = s_rope[b * 64 + jj / 2], sn = s_rope[b * 64 + 32 + jj / 2];
                                    const float e = v0, o = v1;
                                    v0 = e * c - o * sn;
                                    v1 = e * sn + o * c;
                                }
                                if (lane == 0) { out[b * 2 * p.n + 2 * j] = v0; out[b * 2 * p.n + 2 * j + 1] = v1; }
                            }
                        } else if (k == K_C) {
                            const float bo = bs[j];
#pragma unroll
                            for (int b = 0; b < NB; b++)
                                if (lane == 0) out[b * p.n + j] = xs[b * ldD + u] + (acc[0][b] + bo);   // transformer.c:408
                        } else if (k == K_D) {
                            const float bg = bs[j], bu = bs[32 + j];
#pragma unroll
                            for (int b = 0; b < NB; b++) {
                                const float gg = acc[0][b] + bg, up = acc[1][b] + bu;
                                if (lane == 0) out[b * p.n + j] = (gg / (1.0f + expf(-gg))) * up;   // simd.h:394-397
                            }
                        } else {
                            const float lb = bs[j];
#pragma unroll
                            for (int b = 0; b < NB; b++) {
                                const float lg = acc[0][b] + lb;
                                if (lg > bv[b]) { bv[b] = lg; bi[b] = u; }
                                if (a.logits && lane == 0) a.logits[((size_t)t * B + b) * V + u] = lg;
                            }
                        }
                        hs += S_NCW * slots;
                        while (hs >= lo.rs) hs -= lo.rs;
                    }
                    if (k == K_F && lane == 0) {
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            s_best[(cw * MAXB + b) * 2] = bv[b];
                            s_best[(cw * MAXB + b) * 2 + 1] = __builtin_bit_cast(float, bi[b]);
                        }
                    }
                }
                bhead++;
                raw_barrier();                                   // B2: outputs in OUT
            }
        }
        raw_barrier();                                           // B3: stop flag
        if (hd[H_STOP]) { t++; break; }
    }
}

#define DNNHIP_INST5(NB, DC) template __global__ void decode_v5<NB, DC>(StreamArgs);
DNNHIP_INST5(1, 1) DNNHIP_INST5(1, 2) DNNHIP_INST5(1, 3)
DNNHIP_INST5(2, 1) DNNHIP_INST5(2, 2) DNNHIP_INST5(2, 3)

const void *decode_stream_for(int nb, int dc) {
#define DNNHIP_PICK5(NB, DC) if (nb == NB && dc == DC) return reinterpret_cast<const void *>(&decode_v5<NB, DC>);
    DNNHIP_PICK5(1, 1) DNNHIP_PICK5(1, 2) DNNHIP_PICK5(1, 3)
    DNNHIP_PICK5(2, 1) DNNHIP_PICK5(2, 2) DNNHIP_PICK5(2, 3)
    return nullptr;
}

}  // namespace dnnhip
