// decode_kernel.h -- device-side data layout shared by the decode kernel and
// the C-ABI layer (dnn_hip.cpp).  Internal: not part of the public headers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dnnhip {

constexpr int WAVE = 64;          // CDNA wavefront
constexpr int BLOCK = 512;        // threads per workgroup (8 wavefronts, 2 per SIMD)
constexpr int WPB = BLOCK / WAVE;
constexpr int CH = 32;            // cached keys per attention work unit (two half-waves per key)
constexpr int DK = 64;            // head dimension the kernels are built for
constexpr int MAXB = 8;           // batch rows per decode launch
constexpr int MAX_ROWS = 64;      // rows per session (more than MAXB: the batched engine)
constexpr int LDALIGN = 256;      // weight rows / activation rows padded to this many floats
constexpr int FCMAX = 8;          // down-projection input chunks of 256: d_ffn <= 2048
constexpr int PU = 4;             // GEMV rounds of 2-row units a wavefront holds ahead of a phase
constexpr int PE = 2;             // down-projection rounds (rows of d_ffn) held ahead
constexpr int CPW = 2;            // attention chunks a wavefront loads per pass

// GEMV rounds a wavefront holds in registers ahead of a phase, for nb batch
// rows and dc 256-column chunks per row (more rows: fewer held without spills)
constexpr int hold_rounds(int nb, int dc) { return nb >= 8 ? (dc >= 3 ? 1 : 2) : nb >= 4 ? 2 : PU; }

// Workgroup roles of the persistent decode kernel (see plan_roles)
enum { R_AC = 0, R_ATT = 1, R_D = 2, R_E = 3 };

// One transformer block inside the weight arena, as float offsets from its
// base.  Weight matrices are out-major: row n holds the K inputs of output n,
// zero-padded to ld (= K rounded up to LDALIGN).
struct LayerOff {
    uint32_t wqkv;   // [3D][ldD]  rows 0..D-1 = Q, D..2D-1 = K, 2D..3D-1 = V
    uint32_t bqkv;   // [3D]
    uint32_t wo;     // [D][ldD]
    uint32_t bo;     // [D]
    uint32_t g_attn; // [ldD]
    uint32_t g_ffn;  // [ldD]
    uint32_t wgu;    // [F][2][ldD]  gate row f, then up row f
    uint32_t bg;     // [F]
    uint32_t bu;     // [F]
    uint32_t wd;     // [D][ldF]
    uint32_t bd;     // [D]
    float eps_attn, eps_ffn;
};

// Exchange arena: every value one wavefront hands to another travels as an
// 8-byte (value bits, tag) pair written with one coherent (sc1) store; the tag
// is the global step id, so a reader knows a value is this step's by its tag
// and no barrier is needed.  Per layer and batch row:
//   X1 [ldD]  residual stream after attention    X2 [ldD]  after the FFN
//   Q, KN, VN [D]  this step's query and new key/value rows (after RoPE)
//   ATT [D]   merged attention heads            ACT [ldF] SwiGLU output
// then the lm_head argmax partials AMAX [2][B][grid][2] (value, index) and the
// reduced tokens TOK [2][8 copies][16] (one copy per XCD, a cache line each),
// both double buffered by step parity: a step-(t+2) slot is written only after
// the lm_head of step t+2 ran, which needs every workgroup that reads a step-t
// slot to have finished step t+1.  When a head's keys are
// split over ns > 1 workgroups, the attention partials follow, per layer:
//   AO [B*H*ns][DK]  sum_j e^(s_j - m) v_j of record r = (b*H + h)*ns + split
//   AML [B*H*ns][2]  (m, sum_j e^(s_j - m)) of the same record
// and ATT is not used (the out_proj workgroups merge the records).
constexpr int ATT_SPLIT_MAX = 4;  // workgroups per (row, head)
constexpr int ATT_SPLIT_HEADS = 32;  // splitting needs B*H <= this (4 heads per wavefront)
struct Exch {
    int ldD, ldF, D, B, grid, H, ns;
    __host__ __device__ size_t per_row() const { return (size_t)2 * ldD + 4 * (size_t)D + ldF; }
    __host__ __device__ size_t per_layer() const { return per_row() * B; }
    __host__ __device__ size_t base(int l, int b) const { return per_layer() * l + per_row() * b; }
    __host__ __device__ size_t x1(int l, int b) const { return base(l, b); }
    __host__ __device__ size_t x2(int l, int b) const { return base(l, b) + ldD; }
    __host__ __device__ size_t q(int l, int b) const { return base(l, b) + 2 * (size_t)ldD; }
    __host__ __device__ size_t kn(int l, int b) const { return q(l, b) + D; }
    __host__ __device__ size_t vn(int l, int b) const { return q(l, b) + 2 * (size_t)D; }
    __host__ __device__ size_t att(int l, int b) const { return q(l, b) + 3 * (size_t)D; }
    __host__ __device__ size_t act(int l, int b) const { return q(l, b) + 4 * (size_t)D; }
    __host__ __device__ size_t amax(int L, int par, int b, int g) const {
        return per_layer() * L + (((size_t)par * B + b) * grid + g) * 2;
    }
    __host__ __device__ size_t tok(int L, int par, int copy, int b) const {
        return per_layer() * L + (size_t)2 * B * grid * 2 + ((size_t)par * 8 + copy) * 16 + b;
    }
    __host__ __device__ size_t nrec() const { return ns > 1 ? (size_t)B * H * ns : 0; }
    __host__ __device__ size_t ao(int L, int l) const {
        return per_layer() * L + (size_t)2 * B * grid * 2 + 2 * 8 * 16 + (size_t)l * nrec() * (DK + 2);
    }
    __host__ __device__ size_t aml(int L, int l) const { return ao(L, l) + nrec() * DK; }
    __host__ __device__ size_t total(int L) const { return ao(L, L); }
};

struct DecodeArgs {
    int V, D, L, H, F, ldD, ldF;
    const float *wts;       // weight arena: embedding [V][ldD] (also the tied
    uint32_t wts_bytes;     // lm_head), lm_head bias, final gamma, the blocks
    const uint16_t *wts16;  // bf16 copy of the arena's matrices (same element offsets), or null
    uint32_t embed, lm_bias, g_final;   // float offsets in the arena
    const LayerOff *layers; // [L], device
    float eps_final;
    const float *rope;      // [2][rope_rows][DK/2]: cos rows, then sin rows; or null
    int rope_rows;
    int B, max_seq;
    float *kc;              // K^T cache [L][B][H][DK][max_seq], then CH*DK floats of padding
    float *vc;              // V cache   [L][B][H][max_seq][DK], then CH*DK floats of padding
    uint2 *xa;              // exchange arena (Exch layout), pairs
    Exch ex;
    int *pos;               // [B] cached length per row (in/out)
    const int *feed;        // [max n_feed][B]
    const int *n_feed;      // [B]
    int *ids;               // [n_steps][B]
    float *logits;          // [n_steps][B][V] or null
    int n_steps, eos;
    unsigned step0;         // tag of this launch's first step (>= 1, increasing)
    int *err;               // bit 0: a dependency wait hit its spin cap; bit 1: a row had no room
    int *steps_done;
    int seq_limit;          // length + n_steps <= this for every row (max_seq, RoPE rows)
    int n_ac, n_d, n_e;     // workgroups of the A+C, D and E roles (plan_roles); the rest attention
};

// Split of a grid of G workgroups into the kernel's roles: n_ac run the QKV
// and out_proj GEMVs, n_d gate/up, n_e down, and the rest (at least
// min(att_records, G / 5), at least 1) attention.  Among the splits that fit
// -- with every phase's rounds within what a wavefront holds in registers
// (hold; PE for the down rows) where any split allows that -- the one whose
// largest per-wavefront weight share of a phase (rounds x unit length) is
// smallest, then the fewest rounds in total, then the most workgroups; a grid
// too small for that search splits by weight bytes.  Returns false when G
// cannot hold one workgroup per role.
struct Roles {
    int n_ac, n_d, n_e;
};
inline bool plan_roles(int G, int D, int F, int ldD, int ldF, int att_records, Roles &out, int hold = PU) {
    const int n_att = att_records < G / 5 ? (att_records > 1 ? att_records : 1) : (G / 5 > 1 ? G / 5 : 1);
    const int R = G - n_att;
    if (R < 3) return false;
    const int nuA = 3 * D / 2, nuC = D / 2, nuD = F, nuE = D;
    auto cdiv = [](long x, long y) { return (int)((x + y - 1) / y); };
    long best_cost = -1;
    int best_rounds = 0, best_used = 0;
    bool best_held = false;
    for (int ra = 1; ra <= 16; ra++)
        for (int rd = 1; rd <= 32; rd++)
            for (int re = 1; re <= 16; re++) {
                const int nac = cdiv(nuA, (long)WPB * ra), nd = cdiv(nuD, (long)WPB * rd), ne = cdiv(nuE, (long)WPB * re);
                const int used = nac + nd + ne;
                if (used > R) continue;
                const int rc = cdiv(nuC, (long)WPB * nac);
                long cost = (long)ra * 2 * ldD;
                if ((long)rc * 2 * ldD > cost) cost = (long)rc * 2 * ldD;
                if ((long)rd * 2 * ldD > cost) cost = (long)rd * 2 * ldD;
                if ((long)re * ldF > cost) cost = (long)re * ldF;
                const int rounds = ra + rc + rd + re;
                const bool held = ra <= hold && rc <= hold && rd <= hold && re <= PE;
                const bool better = best_cost < 0 || (held && !best_held) ||
                                    (held == best_held &&
                                     (cost < best_cost ||
                                      (cost == best_cost && (rounds < best_rounds || (rounds == best_rounds && used > best_used)))));
                if (better) {
                    best_cost = cost; best_rounds = rounds; best_used = used; best_held = held;
                    out = Roles{nac, nd, ne};
                }
            }
    if (best_cost < 0) {
        // a grid too small for the searched round counts: workgroups in
        // proportion to each role's weight bytes, at least one each (the
        // kernel runs any number of rounds per phase)
        const double wa = ((double)nuA + nuC) * 2 * ldD, wd = (double)nuD * 2 * ldD, we = (double)nuE * ldF;
        const double tot = wa + wd + we;
        int nac = (int)(R * wa / tot), nd = (int)(R * wd / tot);
        if (nac < 1) nac = 1;
        if (nd < 1) nd = 1;
        while (nac + nd > R - 1) {
            if (nac >= nd && nac > 1) nac--;
            else nd--;
        }
        out = Roles{nac, nd, R - nac - nd};
    }
    return true;
}

// Dynamic LDS of the decode kernel (bytes): per-row token / position / done
// flags, per-wavefront argmax and attention partials, the output blocks of PU
// GEMV rounds (OUT [PU][WPB][2*MAXB]), each attention
// wavefront's query and chunk weights (QE [WPB][DK + CPW*CH]), then the staged rows
// XS (layer input), AS (attention), X1S and ACTS, nb rows each.
constexpr int LDS_HEAD_WORDS = 3 * MAXB + 2 * WPB * MAXB + WPB * (DK + 2) + PU * WPB * 2 * MAXB + WPB * (DK + CPW * CH);
inline size_t lds_bytes(int nb, int ldD, int ldF) {
    return (size_t)4 * ((LDS_HEAD_WORDS + 3) / 4 * 4) + (size_t)4 * nb * (3 * (size_t)ldD + ldF);
}

const void *decode_kernel_for(int nb, int dc, bool bf16);

}  // namespace dnnhip
