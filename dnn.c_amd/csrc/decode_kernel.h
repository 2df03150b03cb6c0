// decode_kernel.h -- device-side data layout shared by the decode kernel and
// the C-ABI layer (dnn_hip.cpp).  Internal: not part of the public headers.
#pragma once
#include <hip/hip_runtime.h>

namespace dnnhip {

constexpr int WAVE = 64;          // CDNA wavefront
constexpr int BLOCK = 256;        // threads per workgroup
constexpr int WPB = BLOCK / WAVE; // wavefronts per workgroup
constexpr int NBMAX = 8;          // batch rows per GEMV pass
constexpr int CH = 64;            // cached keys per attention work unit
constexpr int DK = 64;            // head dimension the kernels are built for
constexpr int MAXB = 256;         // batch rows per session
constexpr int LDALIGN = 256;      // out-major weight rows padded to this many floats

// One transformer block in HBM.  All weight matrices are out-major: row n holds
// the K inputs of output n, zero-padded to ld (= K rounded up to LDALIGN).
struct LayerW {
    const float *wqkv;   // [3D][ldD]  rows 0..D-1 = Q, D..2D-1 = K, 2D..3D-1 = V
    const float *bqkv;   // [3D]
    const float *wo;     // [D][ldD]
    const float *bo;     // [D]
    const float *g_attn; // [ldD]
    const float *g_ffn;  // [ldD]
    const float *wgu;    // [F][2][ldD]  gate row f, then up row f
    const float *bg;     // [F]
    const float *bu;     // [F]
    const float *wd;     // [D][ldF]
    const float *bd;     // [D]
    float eps_attn, eps_ffn;
};

struct DecodeArgs {
    int V, D, L, H, F, ldD, ldF;
    const LayerW *layers;   // [L], device
    const float *embed;     // [V][ldD] (also the tied lm_head)
    const float *lm_bias;   // [V]
    const float *g_final;   // [ldD]
    float eps_final;
    const float *rope_cos;  // [rope_rows][DK/2] or null
    const float *rope_sin;
    int B, max_seq, nch_cap;
    float *x;               // [B][ldD] residual stream
    float *q;               // [B][H][DK]
    float *att;             // [B][ldD] merged heads
    float *act;             // [B][ldF] SwiGLU output
    float *kc, *vc;         // [L][B][H][max_seq][DK]
    int *pos;               // [B] cached length per row (in/out)
    float *part;            // [B][H][nch_cap][DK+2] attention partials (m, l, o[DK])
    unsigned *att_cnt;      // [B][H] arrival counters (left at 0)
    float *amax_v;          // [B][grid] per-workgroup argmax partials
    int *amax_i;
    const int *feed;        // [n_feed_max][B]
    const int *n_feed;      // [B]
    int *ids;               // [n_steps][B]
    float *logits;          // [n_steps][B][V] or null
    int n_steps, eos;
    unsigned long long *bar;   // grid barrier: 10 counters, 256 bytes apart
    int *err;               // bit 0: a grid barrier wait hit its spin cap
    int *steps_done;
};

// Dynamic LDS of decode_persistent<nb>: the fixed per-workgroup arrays plus nb
// staged activation rows of ldmax floats.
inline size_t lds_bytes(int nb, int ldmax) {
    return sizeof(float) * (size_t)(3 * WPB * NBMAX + 3 * MAXB) + sizeof(float) * (size_t)nb * ldmax;
}

constexpr size_t BAR_WORDS = 10 * 32;

const void *decode_kernel_for(int nb);

}  // namespace dnnhip
