// decode_lookahead.hip -- the persistent decode kernel for one or two rows.
//
// Same token loop and the same dataflow exchange as decode_v3 (phases A..G,
// tagged values, workgroup-contiguous output blocks), with two changes that
// take the weight stream off the dependency chain:
//
// * Roles.  Wavefront 7 of each workgroup is the stager: it alone polls the
//   exchange (phase inputs, q/k/v of an attention head, argmax partials),
//   copies what it sees into LDS, and writes the workgroup's output blocks.
//   It never has a weight load in flight, so its polls are never queued
//   behind one (vector memory returns in order).  Wavefronts 0..6 compute.
//   Stager and compute wavefronts run separate loops with the same sequence
//   of raw s_barriers (neither role waits for the other's vector memory).
//
// * Layer lookahead.  The per-layer GEMV work is a list of rounds of 7 units
//   (phase E rounds first, then A, C, D); round i belongs to GEMV workgroup
//   i % NG as its slot i / NG (at most 3 slots; E rounds all in slot 0).
//   Each compute wavefront keeps the weights and biases of its unit in every
//   slot in registers and reloads a slot for the next layer right after
//   using it, so a layer's weights stream in while the previous layer's
//   dependency chain runs.  Because vector loads complete in order, a compute
//   wavefront never needs a fresh load while prefetches are in flight: layer
//   offsets, epsilons, RMSNorm gammas and the step's RoPE entries are read
//   from LDS (filled by the stager), and the B*H attention workgroups (the
//   last ones) hold no GEMV slots, so their K/V loads queue behind nothing.
//
// The code avoids reference-capturing lambdas: with them the compiler kept
// closures in scratch memory and read slot state through flat loads, each
// waiting for every prefetch in flight.
//
// The arithmetic of every phase is decode_v3's (same reference citations).

#include "decode_device.h"

namespace dnnhip {

constexpr int NCW = WPB - 1;     // compute wavefronts per workgroup; wavefront NCW stages
constexpr int MAXSLOT = 3;       // GEMV rounds per workgroup per layer

__device__ __forceinline__ void raw_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);     // lgkmcnt(0): this wavefront's LDS traffic is done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

enum { PH_E = 0, PH_A = 1, PH_C = 2, PH_D = 3, PH_NONE = 4 };

// Which phase round i of the layer schedule belongs to, and its round index
// within that phase.  Rounds: E [0, nrE), A [nrE, +nrA), C, D.
struct Sched {
    int nrE, nrA, nrC, nrD;
    __device__ void at(int i, int &ph, int &r) const {
        if (i < nrE) { ph = PH_E; r = i; return; }
        i -= nrE;
        if (i < nrA) { ph = PH_A; r = i; return; }
        i -= nrA;
        if (i < nrC) { ph = PH_C; r = i; return; }
        i -= nrC;
        if (i < nrD) { ph = PH_D; r = i; return; }
        ph = PH_NONE; r = 0;
    }
};

__device__ __forceinline__ bool unit_valid(int ph, int u, int nuA, int nuC, int nuD, int nuE) {
    return ph == PH_E ? u < nuE : ph == PH_A ? u < nuA : ph == PH_C ? u < nuC : ph == PH_D ? u < nuD : false;
}

// Weights and biases of unit u of phase ph (layer offsets lo) into a slot of
// N float4 per lane.  Only a slot of FCMAX entries can hold an E row.
template <int N, int DC>
__device__ __forceinline__ void slot_load(f4 (&w)[N], float (&bs)[2], int ph, int u, const LayerOff &lo, rsrc_t rw,
                                          int ldD, int ldF, int lane) {
    if (N >= FCMAX && ph == PH_E) {
#pragma unroll
        for (int c = 0; c < N; c++)
            if (c * 256 < ldF) w[c] = ld4<CP_NT>(rw, (lo.wd + (size_t)u * ldF + c * 256 + 4 * lane) * 4);
        bs[0] = ld1<0>(rw, (lo.bd + (size_t)u) * 4);
        return;
    }
    size_t row0, b0, b1;
    if (ph == PH_A) { row0 = lo.wqkv + 2 * (size_t)u * ldD; b0 = lo.bqkv + 2 * (size_t)u; b1 = b0 + 1; }
    else if (ph == PH_C) { row0 = lo.wo + 2 * (size_t)u * ldD; b0 = lo.bo + 2 * (size_t)u; b1 = b0 + 1; }
    else { row0 = lo.wgu + 2 * (size_t)u * ldD; b0 = lo.bg + (size_t)u; b1 = lo.bu + (size_t)u; }
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int k = 0; k < DC; k++)
            w[r * DC + k] = ld4<CP_NT>(rw, (row0 + (size_t)r * ldD + k * 256 + 4 * lane) * 4);
    bs[0] = ld1<0>(rw, b0 * 4);
    bs[1] = ld1<0>(rw, b1 * 4);
}

// The two rows of a slot against NB LDS rows at xsrc, each normalised as
// (x * rs) * gamma (norm.c:466-471) when NORM.
template <int N, int NB, int DC, bool NORM>
__device__ __forceinline__ void slot_dot2(const f4 (&w)[N], const float *xsrc, int ldD, const float (&rs)[NB],
                                          const float *gam, int lane, float (&acc)[2][NB]) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float t0 = 0.f, t1 = 0.f;
#pragma unroll
        for (int k = 0; k < DC; k++) {
            f4 y = *reinterpret_cast<const f4 *>(xsrc + b * ldD + k * 256 + 4 * lane);
            if (NORM) {
                const f4 g = *reinterpret_cast<const f4 *>(gam + k * 256 + 4 * lane);
                y.x = (y.x * rs[b]) * g.x; y.y = (y.y * rs[b]) * g.y;
                y.z = (y.z * rs[b]) * g.z; y.w = (y.w * rs[b]) * g.w;
            }
            const f4 a0 = w[k], a1 = w[DC + k];
            t0 += a0.x * y.x + a0.y * y.y + a0.z * y.z + a0.w * y.w;
            t1 += a1.x * y.x + a1.y * y.y + a1.z * y.z + a1.w * y.w;
        }
        acc[0][b] = wave_sum(t0);
        acc[1][b] = wave_sum(t1);
    }
}

// Cached keys / values of the 32-key chunk starting at j0: lanes 0-31 hold
// dims 0-31 of keys j0..j0+31 (K^T rows), lanes 32-63 dims 32-63; vr[jj] is
// dim `lane` of key j0+jj.
__device__ __forceinline__ void kv_chunk_load(float (&kt)[32], float (&vr)[CH], rsrc_t rk, rsrc_t rv, size_t head,
                                              int max_seq, int j0, int half, int kl, int lane) {
    const unsigned kvo = (unsigned)((head + (size_t)(32 * half) * max_seq + j0 + kl) * 4);
    const unsigned vvo = (unsigned)((head + (size_t)j0 * DK + lane) * 4);
#pragma unroll
    for (int i = 0; i < 32; i++) kt[i] = ld1s<CP_SC1>(rk, kvo, (unsigned)(i * max_seq * 4));
#pragma unroll
    for (int jj = 0; jj < CH; jj++) vr[jj] = ld1s<CP_SC1>(rv, vvo, (unsigned)(jj * DK * 4));
}

// Phase F on a compute wavefront: final rms_norm -> tied lm_head + bias ->
// the wavefront's argmax candidates into LDS.  Its two barriers pair with the
// stager's (X2 of the last layer staged; partials written).
template <int NB, int DC>
__device__ __forceinline__ void lm_head_compute(const DecodeArgs &a, rsrc_t rw, const float *xs, const float *gfin,
                                                float eps, float *s_bv, int *s_bi, int t, int G, int g0, int wid,
                                                int lane) {
    const int V = a.V, D = a.D, ldD = a.ldD, B = a.B;
    float bv[NB];
    int bi[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
    const int nu = V / 2;
    const int u0 = g0 * NCW + wid, u1 = (G + g0) * NCW + wid;
    RowUnit<2, DC> U0, U1;
    if (u0 < nu) {
        const size_t bo[2] = {a.lm_bias + 2 * (size_t)u0, a.lm_bias + 2 * (size_t)u0 + 1};
        load_unit<2, DC>(U0, rw, a.embed + 2 * (size_t)u0 * ldD, ldD, bo, lane);
    }
    if (u1 < nu) {
        const size_t bo[2] = {a.lm_bias + 2 * (size_t)u1, a.lm_bias + 2 * (size_t)u1 + 1};
        load_unit<2, DC>(U1, rw, a.embed + 2 * (size_t)u1 * ldD, ldD, bo, lane);
    }
    raw_barrier();                                           // B1: X2 of the last layer staged
    if (u0 < nu) {
        float rs[NB];
        rms_lds<NB, DC>(xs, ldD, D, eps, lane, rs);
        f4 g[DC];
#pragma unroll
        for (int k = 0; k < DC; k++) g[k] = *reinterpret_cast<const f4 *>(gfin + k * 256 + 4 * lane);
        for (int k = 0; (k * G + g0) * NCW + wid < nu; k++) {
            const int u = (k * G + g0) * NCW + wid, v = 2 * u;
            float acc[2][NB];
            float b0, b1;
            if (k == 0) {
                dot_lds<2, NB, DC, true>(U0.w, xs, ldD, rs, g, lane, acc);
                b0 = U0.bias[0]; b1 = U0.bias[1];
            } else if (k == 1) {
                dot_lds<2, NB, DC, true>(U1.w, xs, ldD, rs, g, lane, acc);
                b0 = U1.bias[0]; b1 = U1.bias[1];
            } else {
                const size_t bo[2] = {a.lm_bias + (size_t)v, a.lm_bias + (size_t)v + 1};
                load_unit<2, DC>(U0, rw, a.embed + (size_t)v * ldD, ldD, bo, lane);
                dot_lds<2, NB, DC, true>(U0.w, xs, ldD, rs, g, lane, acc);
                b0 = U0.bias[0]; b1 = U0.bias[1];
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float l0 = acc[0][b] + b0, l1 = acc[1][b] + b1;
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
    raw_barrier();                                           // B2: per-wave partials in LDS
}

__device__ __forceinline__ bool all_rows_done(const DecodeArgs &a, const int *s_done) {
    if (a.eos < 0) return false;
    int all = 1;
    for (int b = 0; b < a.B; b++) all &= s_done[b];
    return all != 0;
}

// One GEMV slot phase on a compute wavefront, for slot arrays w/bs: dot (with
// or without normalisation), epilogue into the LDS output block, reload.
#define SLOT_DOT(S, XSRC, RS, GAM, NORM, ACC, B0, B1)                                                     \
    do {                                                                                                  \
        if ((S) == 0) { slot_dot2<FCMAX, NB, DC, NORM>(w0, XSRC, ldD, RS, GAM, lane, ACC); B0 = bs0[0]; B1 = bs0[1]; } \
        else if ((S) == 1) { slot_dot2<2 * DC, NB, DC, NORM>(w1, XSRC, ldD, RS, GAM, lane, ACC); B0 = bs1[0]; B1 = bs1[1]; } \
        else { slot_dot2<2 * DC, NB, DC, NORM>(w2, XSRC, ldD, RS, GAM, lane, ACC); B0 = bs2[0]; B1 = bs2[1]; } \
    } while (0)
#define SLOT_RELOAD(S, LO)                                                                                \
    do {                                                                                                  \
        if ((S) == 0) slot_load<FCMAX, DC>(w0, bs0, sph[0], u_[0], LO, rw, ldD, ldF, lane);               \
        else if ((S) == 1) slot_load<2 * DC, DC>(w1, bs1, sph[1], u_[1], LO, rw, ldD, ldF, lane);          \
        else slot_load<2 * DC, DC>(w2, bs2, sph[2], u_[2], LO, rw, ldD, ldF, lane);                        \
    } while (0)

template <int NB, int DC>
__global__ void __launch_bounds__(BLOCK)
decode_v4(DecodeArgs a) {
    extern __shared__ float smem[];
    const int ldD = a.ldD, ldF = a.ldF;
    const int B = a.B, D = a.D, H = a.H, F = a.F, V = a.V, Ly = a.L;
    int *s_tok = reinterpret_cast<int *>(smem);                 // [MAXB]
    int *s_pos = s_tok + MAXB;                                  // [MAXB]
    int *s_done = s_pos + MAXB;                                 // [MAXB]
    float *s_bv = reinterpret_cast<float *>(s_done + MAXB);     // [WPB][MAXB]
    int *s_bi = reinterpret_cast<int *>(s_bv + WPB * MAXB);     // [WPB][MAXB]
    float *s_part = reinterpret_cast<float *>(s_bi + WPB * MAXB);   // [WPB][DK + 2]
    float *s_out = s_part + WPB * (DK + 2);                     // [MAXSLOT][WPB][2 * MAXB]
    float *s_qkv = s_out + MAXSLOT * WPB * 2 * MAXB;            // [3][DK]: q, k, v of the head
    float *s_rope = s_qkv + 3 * DK;                             // [WPB][MAXSLOT][MAXB][2] cos, sin
    float *xs = smem + LDS4_HEAD_WORDS;                         // [NB][ldD] layer input (raw)
    float *as = xs + NB * ldD;                                  // [NB][ldD] attention output
    float *x1s = as + NB * ldD;                                 // [NB][ldD] X1 (raw)
    float *acts = x1s + NB * ldD;                               // [NB][ldF] SwiGLU output
    float *sg = acts + NB * ldF;                                // [2L+1][ldD] RMSNorm gammas
    float *s_eps = sg + (2 * Ly + 1) * ldD;                     // [2L+1]
    LayerOff *s_lo = reinterpret_cast<LayerOff *>(s_eps + 2 * Ly + 1);  // [L]

    const int tid = threadIdx.x;
    int lane = tid & (WAVE - 1);
    const int wid = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int G = gridDim.x, g0 = blockIdx.x;
    const int nrows = B < NB ? B : NB;
    Waiter wt{a.err};

    const size_t kv_head = (size_t)DK * a.max_seq;
    const rsrc_t rw = buf(a.wts, a.wts_bytes);
    const rsrc_t xa = buf(a.xa, a.ex.total(Ly) * 8);
    const size_t kv_bytes = ((size_t)Ly * B * H * kv_head + (size_t)CH * DK) * 4;
    const rsrc_t rk = buf(a.kc, kv_bytes);
    const rsrc_t rv = buf(a.vc, kv_bytes);
    const size_t sin_off = (size_t)a.rope_rows * (DK / 2) * 4;
    const rsrc_t rrope = buf(a.rope, a.rope ? 2 * sin_off : 0);
    const size_t xstride = a.ex.per_row();
    const float scale = 1.0f / sqrtf((float)DK);

    const int nuA = 3 * D / 2, nuC = D / 2, nuD = F, nuE = D;
    const Sched sch{(nuE + NCW - 1) / NCW, (nuA + NCW - 1) / NCW, (nuC + NCW - 1) / NCW, (nuD + NCW - 1) / NCW};
    const int NG = G - B * H;                                   // GEMV workgroups; the rest attend
    int sph[MAXSLOT], srd[MAXSLOT];                             // this workgroup's slots (constant-indexed)
#pragma unroll
    for (int s = 0; s < MAXSLOT; s++) {
        sph[s] = PH_NONE; srd[s] = 0;
        if (g0 < NG) sch.at(s * NG + g0, sph[s], srd[s]);
    }
    bool hasA = false, hasC = false, hasD = false, hasE = false;
#pragma unroll
    for (int s = 0; s < MAXSLOT; s++) {
        hasA |= sph[s] == PH_A; hasC |= sph[s] == PH_C; hasD |= sph[s] == PH_D; hasE |= sph[s] == PH_E;
    }
    const int bh = g0 - NG;                                     // attention head of this workgroup
    const bool attn = bh >= 0;

    // ---- launch-wide LDS: zeroed rows, the layer table, every norm's gamma and eps
    for (int i = tid; i < NB * (3 * ldD + ldF); i += BLOCK) xs[i] = 0.f;
    for (int i = tid; i < Ly; i += BLOCK) s_lo[i] = a.layers[i];
    for (int i = tid; i < 2 * Ly + 1; i += BLOCK)
        s_eps[i] = i == 2 * Ly ? a.eps_final : (i & 1) ? a.layers[i / 2].eps_ffn : a.layers[i / 2].eps_attn;
    for (int i = tid; i < (2 * Ly + 1) * ldD; i += BLOCK) {
        const int j = i / ldD, c = i - j * ldD;
        const LayerOff *lp = a.layers + (j < 2 * Ly ? j / 2 : 0);
        const uint32_t off = j == 2 * Ly ? a.g_final : (j & 1) ? lp->g_ffn : lp->g_attn;
        sg[i] = ld1<0>(rw, ((size_t)off + c) * 4);
    }
    for (int b = tid; b < MAXB; b += BLOCK) {
        s_pos[b] = b < B ? a.pos[b] : 0;
        s_done[b] = 0;
        s_tok[b] = 0;
    }
    __syncthreads();

    int t = 0;
    if (wid == NCW) {
        // ================= stager: every poll, every output block
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            if (lane < B && t < a.n_feed[lane]) s_tok[lane] = a.feed[(size_t)t * B + lane];
            // RoPE entries of this step's positions for the compute wavefronts'
            // A units (rope.c:28-32): s_rope[w][s][b] = (cos, sin)
            if (a.rope && !attn) {
                for (int i = lane; i < NCW * MAXSLOT * NB; i += WAVE) {
                    const int w = i / (MAXSLOT * NB), sl = (i / NB) % MAXSLOT, b = i % NB;
                    int ph = PH_NONE, rd = 0;
                    sch.at(sl * NG + g0, ph, rd);
                    const int u = rd * NCW + w, n = 2 * u, sec = n / D;
                    float c = 1.f, sn = 0.f;
                    if (ph == PH_A && u < nuA && sec < 2) {
                        const int j = (n - sec * D) % DK;
                        const size_t ti = ((size_t)s_pos[b < B ? b : B - 1] * (DK / 2) + j / 2) * 4;
                        c = ld1<0>(rrope, ti);
                        sn = ld1<0>(rrope, sin_off + ti);
                    }
                    s_rope[((w * MAXSLOT + sl) * MAXB + b) * 2] = c;
                    s_rope[((w * MAXSLOT + sl) * MAXB + b) * 2 + 1] = sn;
                }
            }
            __syncthreads();                                     // S0
            for (int l = 0; l < Ly; l++) {
                asm volatile("" : "+v"(lane));
                if (!attn) {
                    if (hasA || hasC) {                          // A (and C's residual rows)
                        if (l == 0) {
                            for (int c = 0; c < nrows * (ldD / 256); c++) {   // embedding.c:79-84
                                const int r = c / (ldD / 256), col = (c - r * (ldD / 256)) * 256 + 4 * lane;
                                *reinterpret_cast<f4 *>(xs + r * ldD + col) = ld4<0>(rw, (a.embed + (size_t)s_tok[r] * ldD + col) * 4);
                            }
                        } else {
                            stage_rows_1w<(NB * DC * 2 < 16 ? NB * DC * 2 : 16)>(xs, ldD, D, nrows, a.ex.x2(l - 1, 0), xstride, xa, tag, lane, wt);
                        }
                        raw_barrier();
                        if (hasA) {
                            raw_barrier();
#pragma unroll
                            for (int s = 0; s < MAXSLOT; s++)
                                if (sph[s] == PH_A)
                                    write_block<2, NB, NCW>(s_out + s * (WPB * 2 * MAXB), xa, a.ex.q(l, 0), xstride,
                                                            srd[s] * NCW, nuA, B, tag, lane);
                        }
                    }
                    if (hasC) {
                        stage_rows_1w<(NB * DC * 2 < 16 ? NB * DC * 2 : 16)>(as, ldD, D, nrows, a.ex.att(l, 0), xstride, xa, tag, lane, wt);
                        raw_barrier();
                        raw_barrier();
#pragma unroll
                        for (int s = 0; s < MAXSLOT; s++)
                            if (sph[s] == PH_C)
                                write_block<2, NB, NCW>(s_out + s * (WPB * 2 * MAXB), xa, a.ex.x1(l, 0), xstride,
                                                        srd[s] * NCW, nuC, B, tag, lane);
                    }
                    if (hasD || hasE) {
                        stage_rows_1w<(NB * DC * 2 < 16 ? NB * DC * 2 : 16)>(x1s, ldD, D, nrows, a.ex.x1(l, 0), xstride, xa, tag, lane, wt);
                        raw_barrier();
                        if (hasD) {
                            raw_barrier();
#pragma unroll
                            for (int s = 0; s < MAXSLOT; s++)
                                if (sph[s] == PH_D)
                                    write_block<1, NB, NCW>(s_out + s * (WPB * 2 * MAXB), xa, a.ex.act(l, 0), xstride,
                                                            srd[s] * NCW, nuD, B, tag, lane);
                        }
                    }
                    if (hasE) {
                        stage_rows_1w<16>(acts, ldF, F, nrows, a.ex.act(l, 0), xstride, xa, tag, lane, wt);
                        raw_barrier();
                        raw_barrier();
                        if (sph[0] == PH_E)
                            write_block<1, NB, NCW>(s_out, xa, a.ex.x2(l, 0), xstride, srd[0] * NCW, nuE, B, tag, lane);
                    }
                } else {
                    // B: q, k, v of this workgroup's head -> LDS, then append
                    // position p to the caches and wait until those stores are
                    // complete (barriers do not wait for vector memory)
                    const int b = bh / H, h = bh - b * H, p = s_pos[b];
                    const size_t head = (((size_t)l * B + b) * H + h) * kv_head;
                    float q = 0.f, kn = 0.f, vn = 0.f;
                    wt.reset();
                    for (;;) {
                        const u2 uq = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)((a.ex.q(l, b) + h * DK + lane) * 8), 0, CP_SC1);
                        const u2 uk = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)((a.ex.kn(l, b) + h * DK + lane) * 8), 0, CP_SC1);
                        const u2 uv = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)((a.ex.vn(l, b) + h * DK + lane) * 8), 0, CP_SC1);
                        const unsigned tq = uq.y, tk = uk.y, tv = uv.y;
                        q = as_float(uq.x); kn = as_float(uk.x); vn = as_float(uv.x);
                        if (__all(tq == tag && tk == tag && tv == tag) || !wt.again()) break;
                    }
                    s_qkv[lane] = q; s_qkv[DK + lane] = kn; s_qkv[2 * DK + lane] = vn;
                    st1(rk, (head + (size_t)lane * a.max_seq + p) * 4, kn);    // K^T[d][p]
                    st1(rv, (head + (size_t)p * DK + lane) * 4, vn);           // V[p][d]
                    __builtin_amdgcn_s_waitcnt(0x0f70);                       // vmcnt(0)
                    raw_barrier();
                    raw_barrier();
                }
            }
            // F
            stage_rows_1w<(NB * DC * 2 < 16 ? NB * DC * 2 : 16)>(xs, ldD, D, nrows, a.ex.x2(Ly - 1, 0), xstride, xa, tag, lane, wt);
            raw_barrier();
            raw_barrier();
            if (lane < B) {
                float v = -INFINITY;
                int i = 0x7fffffff;
                for (int ww = 0; ww < NCW; ww++) {
                    const float vv = s_bv[ww * MAXB + lane];
                    const int ii = s_bi[ww * MAXB + lane];
                    if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
                }
                const size_t pa = a.ex.amax(Ly, t & 1, lane, g0);
                put(xa, pa, v, tag);
                put(xa, pa + 1, __builtin_bit_cast(float, i), tag);
            }
            // G: every workgroup's partial -> the next token (the same in all)
            for (int b = 0; b < B; b++) {
                float v = -INFINITY;
                int i = 0x7fffffff;
                for (int gb = 0; gb < G; gb += WAVE) {
                    const int gg = gb + lane;
                    const size_t pa = a.ex.amax(Ly, t & 1, b, gg < G ? gg : 0);
                    u4 qq;
                    wt.reset();
                    for (;;) {
                        qq = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)(pa * 8), 0, CP_SC1);
                        const unsigned t0 = qq.y, t1 = qq.w;
                        if (__all(t0 == tag && t1 == tag) || !wt.again()) break;
                    }
                    const float vv = as_float(qq.x);
                    const int ii = (int)(unsigned)qq.z;
                    if (gg < G && (vv > v || (vv == v && ii < i))) { v = vv; i = ii; }
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
            __syncthreads();                                     // S1
            if (all_rows_done(a, s_done)) { t++; break; }
        }
    } else if (attn) {
        // ================= attention compute wavefronts: phase B of every layer
        float kt[32], vr[CH];
        const int half = lane >> 5, kl = lane & 31;
        const int b = bh / H, h = bh - b * H;
        for (; t < a.n_steps; t++) {
            const unsigned tag = a.step0 + (unsigned)t;
            __syncthreads();                                     // S0
            const int p = s_pos[b], S_ = p + 1, nch = (S_ + CH - 1) / CH;
            for (int l = 0; l < Ly; l++) {
                asm volatile("" : "+v"(lane));
                const size_t head = (((size_t)l * B + b) * H + h) * kv_head;
                if (wid < nch) kv_chunk_load(kt, vr, rk, rv, head, a.max_seq, wid * CH, half, kl, lane);
                raw_barrier();                        // B1: q, k, v in LDS, position p appended
                float m_run = -INFINITY, l_run = 0.f, o_run = 0.f;
                for (int c = wid; c < nch; c += NCW) {
                    const int j0 = c * CH, key = j0 + kl;
                    if (c != wid) kv_chunk_load(kt, vr, rk, rv, head, a.max_seq, j0, half, kl, lane);
                    // keys >= p: stale or neighbouring values, masked by a select
                    float s = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; i++) s += s_qkv[32 * half + i] * (key < p ? kt[i] : 0.f);
                    s += __shfl_xor(s, 32, WAVE);                          // transformer.c:291-297
                    s = s * scale;
                    const bool has_new = p >= j0 && p < j0 + CH;
                    if (has_new) {
                        const float sn = wave_sum(s_qkv[lane] * s_qkv[DK + lane]) * scale;
                        if (key == p) s = sn;
                    }
                    const bool valid = key < S_;
                    const float m_c = wave_max(valid ? s : -INFINITY);
                    const float m_new = fmaxf(m_run, m_c);
                    const float e = valid ? expf(s - m_new) : 0.f;
                    const float fa = expf(m_run - m_new);
                    float o = 0.f;
#pragma unroll
                    for (int jj = 0; jj < CH; jj++) o += bcast(e, jj) * (j0 + jj < p ? vr[jj] : 0.f);
                    if (has_new) o += bcast(e, p - j0) * s_qkv[2 * DK + lane];
                    l_run = l_run * fa + wave_sum(half ? 0.f : e);
                    o_run = o_run * fa + o;
                    m_run = m_new;
                }
                s_part[wid * (DK + 2) + lane] = o_run;
                if (lane == 0) { s_part[wid * (DK + 2) + DK] = m_run; s_part[wid * (DK + 2) + DK + 1] = l_run; }
                raw_barrier();                        // B2: partials in LDS
                if (wid == 0) {
                    float M = -INFINITY;
                    for (int ww = 0; ww < NCW; ww++) M = fmaxf(M, s_part[ww * (DK + 2) + DK]);
                    float O = 0.f, Ls = 0.f;
                    for (int ww = 0; ww < NCW; ww++) {
                        const float mw = s_part[ww * (DK + 2) + DK];
                        const float f = mw == -INFINITY ? 0.f : expf(mw - M);
                        O += s_part[ww * (DK + 2) + lane] * f;
                        Ls += s_part[ww * (DK + 2) + DK + 1] * f;
                    }
                    put(xa, a.ex.att(l, b) + h * DK + lane, O / Ls, tag);
                }
            }
            asm volatile("" : "+v"(lane));
            lm_head_compute<NB, DC>(a, rw, xs, sg + 2 * Ly * ldD, s_eps[2 * Ly], s_bv, s_bi, t, G, g0, wid, lane);
            __syncthreads();                                     // S1
            if (all_rows_done(a, s_done)) { t++; break; }
        }
    } else {
        // ================= GEMV compute wavefronts: phases A, C, D, E
        // Slot weights, reloaded for the next layer right after use.  E rounds
        // come first in the schedule and fit in slot 0 (checked by the host),
        // so only slot 0 holds a full ldF row.
        f4 w0[FCMAX], w1[2 * DC], w2[2 * DC];
        float bs0[2], bs1[2], bs2[2];
        int u_[MAXSLOT];
        bool ok_[MAXSLOT];
#pragma unroll
        for (int s = 0; s < MAXSLOT; s++) {
            u_[s] = srd[s] * NCW + wid;
            ok_[s] = unit_valid(sph[s], u_[s], nuA, nuC, nuD, nuE);
        }
        {
            const LayerOff lo = load_layer(s_lo);
#pragma unroll
            for (int s = 0; s < MAXSLOT; s++)
                if (ok_[s]) SLOT_RELOAD(s, lo);
        }
        for (; t < a.n_steps; t++) {
            __syncthreads();                                     // S0
            for (int l = 0; l < Ly; l++) {
                asm volatile("" : "+v"(lane));
                const float *g_attn = sg + (2 * l) * ldD, *g_ffn = sg + (2 * l + 1) * ldD;
                const LayerOff lo_next = load_layer(s_lo + (l + 1 < Ly ? l + 1 : 0));
                // ---- A: rms_norm -> qkv + bias -> RoPE -> Q / KN / VN
                if (hasA || hasC) {
                    raw_barrier();                               // B1: layer input in XS
                    if (hasA) {
                        float rs[NB];
                        rms_lds<NB, DC>(xs, ldD, D, s_eps[2 * l], lane, rs);
#pragma unroll
                        for (int s = 0; s < MAXSLOT; s++) {
                            if (sph[s] != PH_A || !ok_[s]) continue;
                            const int sec = 2 * u_[s] / D;
                            float acc[2][NB];
                            float b0, b1;
                            SLOT_DOT(s, xs, rs, g_attn, true, acc, b0, b1);
                            float *out = s_out + s * (WPB * 2 * MAXB);
#pragma unroll
                            for (int b = 0; b < NB; b++) {
                                float v0 = acc[0][b] + b0, v1 = acc[1][b] + b1;
                                if (sec < 2 && a.rope) {             // rope.c:28-32
                                    const float c = s_rope[((wid * MAXSLOT + s) * MAXB + b) * 2];
                                    const float sn = s_rope[((wid * MAXSLOT + s) * MAXB + b) * 2 + 1];
                                    const float e = v0, o = v1;
                                    v0 = e * c - o * sn;
                                    v1 = e * sn + o * c;
                                }
                                if (lane == 0) { out[wid * NB * 2 + b * 2] = v0; out[wid * NB * 2 + b * 2 + 1] = v1; }
                            }
                            SLOT_RELOAD(s, lo_next);
                        }
                        raw_barrier();                           // B2: outputs in LDS
                    }
                }
                // ---- C: out_proj + bias + residual -> X1 (transformer.c:408)
                if (hasC) {
                    raw_barrier();
                    float rs[NB];
#pragma unroll
                    for (int s = 0; s < MAXSLOT; s++) {
                        if (sph[s] != PH_C || !ok_[s]) continue;
                        const int n = 2 * u_[s];
                        float acc[2][NB];
                        float b0, b1;
                        SLOT_DOT(s, as, rs, nullptr, false, acc, b0, b1);
                        float *out = s_out + s * (WPB * 2 * MAXB);
                        if (lane == 0) {
#pragma unroll
                            for (int b = 0; b < NB; b++) {
                                out[wid * NB * 2 + b * 2] = xs[b * ldD + n] + (acc[0][b] + b0);
                                out[wid * NB * 2 + b * 2 + 1] = xs[b * ldD + n + 1] + (acc[1][b] + b1);
                            }
                        }
                        SLOT_RELOAD(s, lo_next);
                    }
                    raw_barrier();
                }
                // ---- D: rms_norm(X1) -> gate/up + bias -> SwiGLU -> ACT (nn.c:61-78, simd.h:394-397)
                if (hasD || hasE) {
                    raw_barrier();
                    if (hasD) {
                        float rs[NB];
                        rms_lds<NB, DC>(x1s, ldD, D, s_eps[2 * l + 1], lane, rs);
#pragma unroll
                        for (int s = 0; s < MAXSLOT; s++) {
                            if (sph[s] != PH_D || !ok_[s]) continue;
                            float acc[2][NB];
                            float b0, b1;
                            SLOT_DOT(s, x1s, rs, g_ffn, true, acc, b0, b1);
                            float *out = s_out + s * (WPB * 2 * MAXB);
                            if (lane == 0) {
#pragma unroll
                                for (int b = 0; b < NB; b++) {
                                    const float gg = acc[0][b] + b0, up = acc[1][b] + b1;
                                    out[wid * NB + b] = (gg / (1.0f + expf(-gg))) * up;
                                }
                            }
                            SLOT_RELOAD(s, lo_next);
                        }
                        raw_barrier();
                    }
                }
                // ---- E: down + bias + residual -> X2 (transformer.c:415)
                if (hasE) {
                    raw_barrier();
                    if (sph[0] == PH_E && ok_[0]) {
                        const int n = u_[0];
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            float sum = 0.f;
#pragma unroll
                            for (int c = 0; c < FCMAX; c++) {
                                if (c * 256 >= ldF) continue;
                                const f4 y = *reinterpret_cast<const f4 *>(acts + b * ldF + c * 256 + 4 * lane);
                                sum += w0[c].x * y.x + w0[c].y * y.y + w0[c].z * y.z + w0[c].w * y.w;
                            }
                            sum = wave_sum(sum);
                            if (lane == 0) s_out[wid * NB + b] = x1s[b * ldD + n] + (sum + bs0[0]);
                        }
                        slot_load<FCMAX, DC>(w0, bs0, sph[0], u_[0], lo_next, rw, ldD, ldF, lane);
                    }
                    raw_barrier();
                }
            }
            asm volatile("" : "+v"(lane));
            lm_head_compute<NB, DC>(a, rw, xs, sg + 2 * Ly * ldD, s_eps[2 * Ly], s_bv, s_bi, t, G, g0, wid, lane);
            __syncthreads();                                     // S1
            if (all_rows_done(a, s_done)) { t++; break; }
        }
    }
    if (g0 == 0 && tid < B) a.pos[tid] = s_pos[tid];
    if (g0 == 0 && tid == 0) *a.steps_done = t;
}

#undef SLOT_DOT
#undef SLOT_RELOAD

#define DNNHIP_INST4(NB, DC) template __global__ void decode_v4<NB, DC>(DecodeArgs);
DNNHIP_INST4(1, 1) DNNHIP_INST4(1, 2) DNNHIP_INST4(1, 3)
DNNHIP_INST4(2, 1) DNNHIP_INST4(2, 2) DNNHIP_INST4(2, 3)

const void *decode_lookahead_for(int nb, int dc) {
#define DNNHIP_PICK4(NB, DC) if (nb == NB && dc == DC) return reinterpret_cast<const void *>(&decode_v4<NB, DC>);
    DNNHIP_PICK4(1, 1) DNNHIP_PICK4(1, 2) DNNHIP_PICK4(1, 3)
    DNNHIP_PICK4(2, 1) DNNHIP_PICK4(2, 2) DNNHIP_PICK4(2, 3)
    return nullptr;
}

}  // namespace dnnhip
