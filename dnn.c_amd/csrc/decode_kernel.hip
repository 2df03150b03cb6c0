// decode_kernel.hip -- the persistent gfx950 decode kernel.
//
// One launch runs n_steps of the GPT token loop of masc-it/dnn.c
// (decoder_lm_generate, gpt.c:306-375) for B <= 8 rows at once:
//
//   per layer (transformer_block_forward_cached_ex, transformer.c:211-416)
//     A  rms_norm(x) -> qkv GEMV + bias -> RoPE(q, k) -> Q / KN / VN, K and V cache rows
//     B  split-S attention over the row's S = pos+1 keys (one 64-key chunk per
//        wavefront), then a combine of the chunks' (o, max, sum) partials
//     C  out_proj GEMV + bias + residual                      -> X1
//     D  rms_norm(X1) -> gate/up GEMV + bias -> SwiGLU        -> ACT
//     E  down GEMV + bias + residual                          -> X2
//   then
//     F  rms_norm(X2) -> tied lm_head GEMV + bias -> argmax partial per workgroup
//     G  every workgroup reduces the partials (first index of the maximum,
//        gpt.c:220-230) and feeds the token to the next step's embedding rows
//
// Synchronisation is dataflow, not barriers.  Every value a wavefront produces
// for others is one 8-byte (value, tag) store with device-coherent (sc1)
// caching; the tag is the global step id.  A consumer polls the values it needs
// until all carry this step's tag, so each dependency costs one coherent hop
// (~0.7 us on MI355X) and no L2 writeback/invalidate is ever issued.  A
// wavefront issues the weight loads of its next work unit before it polls that
// unit's inputs, so weight streaming overlaps the wait.
//
// Weights are out-major (row n = the K inputs of output n, padded to a multiple
// of 256 floats): each output is one contiguous, coalesced dot product owned by
// one wavefront.  Every memory access goes through a buffer descriptor sized to
// its tensor, so the hardware range-checks it (out-of-range loads read 0,
// stores are dropped).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include "decode_kernel.h"

namespace dnnhip {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int CP_NT = 2;        // streaming (non-temporal): weights, read once per step
constexpr int CP_SC1 = 16;      // device-coherent: everything written inside the launch
constexpr unsigned SPIN_CAP = 1u << 22;
constexpr int FCMAX = 8;        // down-projection K chunks held per pass

// Bit reinterpretation through a by-value scalar: clang miscompiles
// __builtin_bit_cast applied directly to an ext-vector element (q.z reads q.x).
__device__ __forceinline__ float as_float(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ unsigned as_uint(float f) { return __builtin_bit_cast(unsigned, f); }

__device__ __forceinline__ rsrc_t buf(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes < 0x7fffffffu ? bytes : 0x7fffffffu), 0x00020000);
}
template <int CP>
__device__ __forceinline__ f4 ld4(rsrc_t r, size_t off) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)off, 0, CP));
}
template <int CP>
__device__ __forceinline__ float ld1(rsrc_t r, size_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (unsigned)off, 0, CP));
}
__device__ __forceinline__ void st1(rsrc_t r, size_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (unsigned)off, 0, CP_SC1);
}
__device__ __forceinline__ void put(rsrc_t xa, size_t pair, float v, unsigned tag) {
    u2 w = {__builtin_bit_cast(unsigned, v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(w, xa, (unsigned)(pair * 8), 0, CP_SC1);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}
__device__ __forceinline__ float bcast(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Bounded wait bookkeeping: once any wait gives up, err[0] is set and every
// later wait returns at once, so all waves run to the end of the launch.
struct Waiter {
    int *err;
    bool dead = false;
    unsigned it = 0;
    __device__ bool again() {
        if (dead) return false;
        if ((++it & 63u) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) { dead = true; return false; }
        if (it >= SPIN_CAP) { atomicOr(err, 1); dead = true; return false; }
        __builtin_amdgcn_s_sleep(1);
        return true;
    }
    __device__ void reset() { it = 0; }
};

// One row of n valid values, tagged, starting at pair index `base`: lane holds
// columns k*256 + 4*lane + j (k < NC, j < 4).  Spins until all carry `tag`.
template <int NC>
__device__ __forceinline__ void poll_row(rsrc_t xa, size_t base, int n, unsigned tag, int lane, float *v, Waiter &w) {
    w.reset();
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < NC; k++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int col = k * 256 + 4 * lane + 2 * h;
                const u4 q = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)((base + col) * 8), 0, CP_SC1);
                v[k * 4 + 2 * h] = as_float(q.x);
                v[k * 4 + 2 * h + 1] = as_float(q.z);
                ok &= (col >= n || q.y == tag) && (col + 1 >= n || q.w == tag);
            }
        }
        if (__all(ok) || !w.again()) return;
    }
}

// A single tagged value per lane at pair index `p` (p < 0: nothing to wait for).
__device__ __forceinline__ float poll1(rsrc_t xa, long p, unsigned tag, Waiter &w) {
    w.reset();
    for (;;) {
        u2 q = {0u, tag};
        if (p >= 0) q = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)(p * 8), 0, CP_SC1);
        if (__all(q.y == tag) || !w.again()) return as_float(q.x);
    }
}

// rms_norm over lane-held row slices (norm.c:433-440, 466-471):
// y = (x * rs) * gamma, rs = 1/sqrtf(sum(x^2) * (1/n) + eps).
template <int NB, int DC>
__device__ __forceinline__ void rms_rows(float (&x)[NB][DC * 4], rsrc_t rw, size_t g_off, int n, float eps, int lane) {
    float g[DC * 4];
#pragma unroll
    for (int k = 0; k < DC; k++) {
        const f4 t = ld4<0>(rw, (g_off + k * 256 + 4 * lane) * 4);
        g[4 * k] = t.x; g[4 * k + 1] = t.y; g[4 * k + 2] = t.z; g[4 * k + 3] = t.w;
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < DC * 4; i++) ss += x[b][i] * x[b][i];
        ss = wave_sum(ss);
        const float rs = 1.0f / sqrtf(ss * (1.0f / (float)n) + eps);
#pragma unroll
        for (int i = 0; i < DC * 4; i++) x[b][i] = (x[b][i] * rs) * g[i];
    }
}

// weights of R consecutive out-major rows starting at float offset `off` in the
// arena (row stride ld floats), DC chunks of 256 columns each
template <int R, int DC>
__device__ __forceinline__ void load_rows(f4 (&w)[R][DC], rsrc_t rw, size_t off, int ld, int lane) {
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int k = 0; k < DC; k++) w[r][k] = ld4<CP_NT>(rw, (off + (size_t)r * ld + k * 256 + 4 * lane) * 4);
}

template <int R, int NB, int DC>
__device__ __forceinline__ void dot_rows(const f4 (&w)[R][DC], const float (&x)[NB][DC * 4], float (&acc)[R][NB]) {
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < DC; k++)
                s += w[r][k].x * x[b][4 * k] + w[r][k].y * x[b][4 * k + 1] + w[r][k].z * x[b][4 * k + 2] + w[r][k].w * x[b][4 * k + 3];
            acc[r][b] = wave_sum(s);
        }
}

// Activation rows of a GEMV input.  `which`: 0 = layer input (the embedding row
// of this step's token at layer 0, else X2 of the layer below), 1 = X1,
// 2 = ATT, 3 = X2 of the last layer.
template <int NB, int DC>
__device__ __forceinline__ void load_input(float (&x)[NB][DC * 4], const DecodeArgs &a, rsrc_t xa, rsrc_t rw,
                                           const int *s_tok, int which, int l, unsigned tag, int lane, Waiter &wt) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int bb = b < a.B ? b : a.B - 1;
        if (which == 0 && l == 0) {
#pragma unroll
            for (int k = 0; k < DC; k++) {
                const f4 t = ld4<0>(rw, (a.embed + (size_t)s_tok[bb] * a.ldD + k * 256 + 4 * lane) * 4);
                x[b][4 * k] = t.x; x[b][4 * k + 1] = t.y; x[b][4 * k + 2] = t.z; x[b][4 * k + 3] = t.w;
            }
        } else {
            size_t base;
            if (which == 0) base = a.ex.x2(l - 1, bb);
            else if (which == 1) base = a.ex.x1(l, bb);
            else if (which == 2) base = a.ex.att(l, bb);
            else base = a.ex.x2(a.L - 1, bb);
            poll_row<DC>(xa, base, a.D, tag, lane, x[b], wt);
        }
    }
}

template <int NB, int DC>
__global__ void __launch_bounds__(BLOCK)
decode_v2(DecodeArgs a) {
    extern __shared__ int smem[];
    int *s_tok = smem;                                          // [MAXB]
    int *s_pos = s_tok + MAXB;                                  // [MAXB]
    int *s_done = s_pos + MAXB;                                 // [MAXB]
    float *s_bv = reinterpret_cast<float *>(s_done + MAXB);     // [WPB][MAXB]
    int *s_bi = reinterpret_cast<int *>(s_bv + WPB * MAXB);     // [WPB][MAXB]

    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
    const int gw = blockIdx.x * WPB + wid, nw = gridDim.x * WPB;
    const int B = a.B, D = a.D, H = a.H, F = a.F, ldD = a.ldD, ldF = a.ldF, V = a.V;
    Waiter wt{a.err};

    const size_t kv_head = (size_t)DK * a.max_seq;              // floats per (layer, row, head)
    const rsrc_t rw = buf(a.wts, a.wts_bytes);
    const rsrc_t xa = buf(a.xa, a.ex.total(a.L) * 8);
    const rsrc_t rk = buf(a.kc, (size_t)a.L * B * H * kv_head * 4);
    const rsrc_t rv = buf(a.vc, (size_t)a.L * B * H * kv_head * 4);
    const size_t sin_off = (size_t)a.rope_rows * (DK / 2) * 4;      // bytes
    const rsrc_t rrope = buf(a.rope, a.rope ? 2 * sin_off : 0);
    const float scale = 1.0f / sqrtf((float)DK);

    for (int b = tid; b < MAXB; b += BLOCK) {
        s_pos[b] = b < B ? a.pos[b] : 0;
        s_done[b] = 0;
        s_tok[b] = 0;
    }
    __syncthreads();

    int t = 0;
    for (; t < a.n_steps; t++) {
        const unsigned tag = a.step0 + (unsigned)t;
        for (int b = tid; b < B; b += BLOCK)
            if (t < a.n_feed[b]) s_tok[b] = a.feed[(size_t)t * B + b];
        __syncthreads();
        int max_s = 0;
        for (int b = 0; b < B; b++) max_s = max(max_s, s_pos[b] + 1);
        const int nch_max = (max_s + CH - 1) / CH;

        for (int l = 0; l < a.L; l++) {
            const LayerOff w = a.layers[l];

            // ---- A: rms_norm -> qkv + bias -> RoPE -> Q / KN / VN and the cache rows
            {
                const int nu = 3 * D / 2;            // RoPE pairs (2k, 2k+1) stay in one wavefront
                if (gw < nu) {
                    f4 wr[2][DC];
                    load_rows<2, DC>(wr, rw, w.wqkv + 2 * (size_t)gw * ldD, ldD, lane);
                    float x[NB][DC * 4];
                    load_input<NB, DC>(x, a, xa, rw, s_tok, 0, l, tag, lane, wt);
                    rms_rows<NB, DC>(x, rw, w.g_attn, D, w.eps_attn, lane);
                    for (int u = gw;;) {
                        const int n = 2 * u;
                        float acc[2][NB];
                        dot_rows<2, NB, DC>(wr, x, acc);
                        const int sec = n / D, within = n - sec * D, h = within / DK, j = within - h * DK;
                        const float b0 = ld1<0>(rw, (w.bqkv + (size_t)n) * 4), b1 = ld1<0>(rw, (w.bqkv + (size_t)n + 1) * 4);
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            if (b >= B || lane != 0) continue;
                            float v0 = acc[0][b] + b0, v1 = acc[1][b] + b1;
                            const int p = s_pos[b];
                            if (sec < 2 && a.rope) {     // rope.c:28-32
                                const size_t ti = ((size_t)p * (DK / 2) + j / 2) * 4;
                                const float c = ld1<0>(rrope, ti), s = ld1<0>(rrope, sin_off + ti);
                                const float e = v0, o = v1;
                                v0 = e * c - o * s;
                                v1 = e * s + o * c;
                            }
                            const size_t dst = (sec == 0 ? a.ex.q(l, b) : sec == 1 ? a.ex.kn(l, b) : a.ex.vn(l, b)) + h * DK + j;
                            put(xa, dst, v0, tag);
                            put(xa, dst + 1, v1, tag);
                        }
                        u += nw;
                        if (u >= nu) break;
                        load_rows<2, DC>(wr, rw, w.wqkv + 2 * (size_t)u * ldD, ldD, lane);
                    }
                }
            }

            // ---- B: attention, one 32-key chunk of one (row, head) per wavefront.
            // Scores: lanes 0-31 hold dims 0-31, lanes 32-63 dims 32-63 of the
            // chunk's 32 keys (key = j0 + (lane & 31)); P.V: lane = output dim.
            {
                const int nu = B * H * nch_max;
                const int half = lane >> 5, kl = lane & 31;
                for (int u = gw; u < nu; u += nw) {
                    const int c = u % nch_max, bh = u / nch_max, b = bh / H, h = bh - b * H;
                    const int p = s_pos[b], S = p + 1, nch = (S + CH - 1) / CH;
                    if (c >= nch) continue;
                    const int j0 = c * CH, key = j0 + kl;
                    const size_t head = (((size_t)l * B + b) * H + h) * kv_head;
                    // cached keys (positions < p) of this chunk, issued before the waits
                    // (unconditional loads, then a select: keys >= p hold stale or
                    // neighbouring values, all finite, never used unmasked)
                    float kt[32], vr[CH];
#pragma unroll
                    for (int i = 0; i < 32; i++) {
                        const float t = ld1<CP_SC1>(rk, (head + (size_t)(32 * half + i) * a.max_seq + key) * 4);
                        kt[i] = key < p ? t : 0.f;
                    }
#pragma unroll
                    for (int jj = 0; jj < CH; jj++) {
                        const float t = ld1<CP_SC1>(rv, (head + (size_t)(j0 + jj) * DK + lane) * 4);
                        vr[jj] = j0 + jj < p ? t : 0.f;
                    }
                    const float q = poll1(xa, (long)(a.ex.q(l, b) + h * DK + lane), tag, wt);
                    const bool has_new = p >= j0 && p < j0 + CH;
                    float kn = 0.f, vn = 0.f;
                    if (has_new) {
                        kn = poll1(xa, (long)(a.ex.kn(l, b) + h * DK + lane), tag, wt);
                        vn = poll1(xa, (long)(a.ex.vn(l, b) + h * DK + lane), tag, wt);
                    }
                    if (has_new) {
                        // the wavefront owning position p appends it to the caches;
                        // its s_waitcnt before the output store below orders these
                        // stores before every later step's reads of them
                        st1(rk, (head + (size_t)lane * a.max_seq + p) * 4, kn);    // K^T[d][p]
                        st1(rv, (head + (size_t)p * DK + lane) * 4, vn);           // V[p][d]
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
                    const float m = wave_max(valid ? s : -INFINITY);
                    const float e = valid ? expf(s - m) : 0.f;
                    const float lsum = wave_sum(half ? 0.f : e);
                    float o = 0.f;
#pragma unroll
                    for (int jj = 0; jj < CH; jj++) o += bcast(e, jj) * vr[jj];
                    if (has_new) {
                        o += bcast(e, p - j0) * vn;
                        __builtin_amdgcn_s_waitcnt(0x0f70);     // vmcnt(0): the cache stores are complete
                    }
                    if (nch == 1) {
                        put(xa, a.ex.att(l, b) + h * DK + lane, o / lsum, tag);
                    } else {
                        const size_t pp = a.ex.part(l, b, h, c);
                        put(xa, pp + lane, o, tag);
                        if (lane == 0) { put(xa, pp + DK, m, tag); put(xa, pp + DK + 1, lsum, tag); }
                    }
                }
                // combine the chunks of each (row, head): max-rescaled sums
                for (int u = gw; u < B * H; u += nw) {
                    const int b = u / H, h = u - b * H;
                    const int S = s_pos[b] + 1, nch = (S + CH - 1) / CH;
                    if (nch == 1) continue;
                    float M = -INFINITY, Ls = 0.f, O = 0.f;
                    for (int c = 0; c < nch; c++) {
                        const size_t pp = a.ex.part(l, b, h, c);
                        const float oc = poll1(xa, (long)(pp + lane), tag, wt);
                        const float mc = poll1(xa, (long)(pp + DK), tag, wt);
                        const float lc = poll1(xa, (long)(pp + DK + 1), tag, wt);
                        const float Mn = fmaxf(M, mc);
                        const float fa = expf(M - Mn), fb = expf(mc - Mn);
                        O = O * fa + oc * fb;
                        Ls = Ls * fa + lc * fb;
                        M = Mn;
                    }
                    put(xa, a.ex.att(l, b) + h * DK + lane, O / Ls, tag);
                }
            }

            // ---- C: out_proj + bias + residual -> X1
            {
                const int nu = D / 2;
                if (gw < nu) {
                    f4 wr[2][DC];
                    load_rows<2, DC>(wr, rw, w.wo + 2 * (size_t)gw * ldD, ldD, lane);
                    float x[NB][DC * 4];
                    load_input<NB, DC>(x, a, xa, rw, s_tok, 2, l, tag, lane, wt);
                    for (int u = gw;;) {
                        const int n = 2 * u;
                        float acc[2][NB];
                        dot_rows<2, NB, DC>(wr, x, acc);
                        const float bias = ld1<0>(rw, (w.bo + (size_t)n + (lane & 1)) * 4);
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            if (b >= B) continue;
                            // residual in (lanes 0, 1): embedding row at layer 0, else X2 of the layer below
                            float r = 0.f;
                            if (l == 0) {
                                if (lane < 2) r = ld1<0>(rw, (a.embed + (size_t)s_tok[b] * ldD + n + lane) * 4);
                            } else {
                                r = poll1(xa, lane < 2 ? (long)(a.ex.x2(l - 1, b) + n + lane) : -1L, tag, wt);
                            }
                            const float y = (lane == 0 ? acc[0][b] : acc[1][b]) + bias;
                            if (lane < 2) put(xa, a.ex.x1(l, b) + n + lane, r + y, tag);   // transformer.c:408
                        }
                        u += nw;
                        if (u >= nu) break;
                        load_rows<2, DC>(wr, rw, w.wo + 2 * (size_t)u * ldD, ldD, lane);
                    }
                }
            }

            // ---- D: rms_norm(X1) -> gate/up + bias -> SwiGLU -> ACT  (nn.c:61-78, simd.h:394-397)
            {
                const int nu = F;
                if (gw < nu) {
                    f4 wr[2][DC];
                    load_rows<2, DC>(wr, rw, w.wgu + 2 * (size_t)gw * ldD, ldD, lane);
                    float x[NB][DC * 4];
                    load_input<NB, DC>(x, a, xa, rw, s_tok, 1, l, tag, lane, wt);
                    rms_rows<NB, DC>(x, rw, w.g_ffn, D, w.eps_ffn, lane);
                    for (int f = gw;;) {
                        float acc[2][NB];
                        dot_rows<2, NB, DC>(wr, x, acc);
                        const float bgf = ld1<0>(rw, (w.bg + (size_t)f) * 4), bup = ld1<0>(rw, (w.bu + (size_t)f) * 4);
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            if (b >= B || lane != 0) continue;
                            const float g = acc[0][b] + bgf, up = acc[1][b] + bup;
                            put(xa, a.ex.act(l, b) + f, (g / (1.0f + expf(-g))) * up, tag);
                        }
                        f += nw;
                        if (f >= nu) break;
                        load_rows<2, DC>(wr, rw, w.wgu + 2 * (size_t)f * ldD, ldD, lane);
                    }
                }
            }

            // ---- E: down + bias + residual -> X2
            {
                const int nu = D, FC = ldF / 256;
                for (int n = gw; n < nu; n += nw) {
                    float acc[NB];
#pragma unroll
                    for (int b = 0; b < NB; b++) acc[b] = 0.f;
                    for (int k0 = 0; k0 < FC; k0 += FCMAX) {
                        f4 wr[FCMAX];
#pragma unroll
                        for (int k = 0; k < FCMAX; k++)
                            if (k0 + k < FC) wr[k] = ld4<CP_NT>(rw, (w.wd + (size_t)n * ldF + (k0 + k) * 256 + 4 * lane) * 4);
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            const int bb = b < B ? b : B - 1;
                            float xv[FCMAX * 4];
                            wt.reset();
                            for (;;) {
                                bool ok = true;
#pragma unroll
                                for (int k = 0; k < FCMAX; k++) {
                                    if (k0 + k >= FC) continue;
#pragma unroll
                                    for (int hh = 0; hh < 2; hh++) {
                                        const int col = (k0 + k) * 256 + 4 * lane + 2 * hh;
                                        const u4 q = __builtin_amdgcn_raw_buffer_load_b128(
                                            xa, (unsigned)((a.ex.act(l, bb) + col) * 8), 0, CP_SC1);
                                        xv[4 * k + 2 * hh] = as_float(q.x);
                                        xv[4 * k + 2 * hh + 1] = as_float(q.z);
                                        ok &= (col >= F || q.y == tag) && (col + 1 >= F || q.w == tag);
                                    }
                                }
                                if (__all(ok) || !wt.again()) break;
                            }
                            float s = 0.f;
#pragma unroll
                            for (int k = 0; k < FCMAX; k++)
                                if (k0 + k < FC)
                                    s += wr[k].x * xv[4 * k] + wr[k].y * xv[4 * k + 1] + wr[k].z * xv[4 * k + 2] + wr[k].w * xv[4 * k + 3];
                            acc[b] += s;
                        }
                    }
                    const float bdn = ld1<0>(rw, (w.bd + (size_t)n) * 4);
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        if (b >= B) continue;
                        const float y = wave_sum(acc[b]) + bdn;
                        const float r = poll1(xa, lane == 0 ? (long)(a.ex.x1(l, b) + n) : -1L, tag, wt);
                        if (lane == 0) put(xa, a.ex.x2(l, b) + n, r + y, tag);        // transformer.c:415
                    }
                }
            }
        }

        // ---- F: final rms_norm -> tied lm_head + bias -> per-workgroup argmax
        {
            float bv[NB];
            int bi[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
            const int nu = V / 2;
            if (gw < nu) {
                f4 wr[2][DC];
                load_rows<2, DC>(wr, rw, a.embed + 2 * (size_t)gw * ldD, ldD, lane);
                float x[NB][DC * 4];
                load_input<NB, DC>(x, a, xa, rw, s_tok, 3, 0, tag, lane, wt);
                rms_rows<NB, DC>(x, rw, a.g_final, D, a.eps_final, lane);
                for (int u = gw;;) {
                    const int v = 2 * u;
                    float acc[2][NB];
                    dot_rows<2, NB, DC>(wr, x, acc);
                    const float l0b = ld1<0>(rw, (a.lm_bias + (size_t)v) * 4), l1b = ld1<0>(rw, (a.lm_bias + (size_t)v + 1) * 4);
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const float l0 = acc[0][b] + l0b, l1 = acc[1][b] + l1b;
                        if (l0 > bv[b]) { bv[b] = l0; bi[b] = v; }
                        if (l1 > bv[b]) { bv[b] = l1; bi[b] = v + 1; }
                        if (a.logits && b < B && lane < 2)
                            a.logits[((size_t)t * B + b) * V + v + lane] = lane == 0 ? l0 : l1;
                    }
                    u += nw;
                    if (u >= nu) break;
                    load_rows<2, DC>(wr, rw, a.embed + 2 * (size_t)u * ldD, ldD, lane);
                }
            }
            if (lane == 0) {
#pragma unroll
                for (int b = 0; b < NB; b++) { s_bv[wid * MAXB + b] = bv[b]; s_bi[wid * MAXB + b] = bi[b]; }
            }
            __syncthreads();
            if (tid < B) {
                float v = -INFINITY;
                int i = 0x7fffffff;
                for (int ww = 0; ww < WPB; ww++) {
                    const float vv = s_bv[ww * MAXB + tid];
                    const int ii = s_bi[ww * MAXB + tid];
                    if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
                }
                const size_t pa = a.ex.amax(a.L, t & 1, tid, blockIdx.x);
                put(xa, pa, v, tag);
                put(xa, pa + 1, __builtin_bit_cast(float, i), tag);
            }
        }

        // ---- G: every workgroup reduces the partials -> next token (same in all)
        if (wid == 0) {
            for (int b = 0; b < B; b++) {
                float v = -INFINITY;
                int i = 0x7fffffff;
                for (int g0 = 0; g0 < (int)gridDim.x; g0 += WAVE) {
                    const int g = g0 + lane;
                    const long pv = g < (int)gridDim.x ? (long)a.ex.amax(a.L, t & 1, b, g) : -1L;
                    const float vv = poll1(xa, pv, tag, wt);
                    const float iv = poll1(xa, pv >= 0 ? pv + 1 : -1L, tag, wt);
                    const int ii = __builtin_bit_cast(int, iv);
                    if (pv >= 0 && (vv > v || (vv == v && ii < i))) { v = vv; i = ii; }
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
                    if (blockIdx.x == 0) a.ids[(size_t)t * B + b] = i;
                }
            }
        }
        __syncthreads();
        if (a.eos >= 0) {
            int all = 1;
            for (int b = 0; b < B; b++) all &= s_done[b];
            if (all) { t++; break; }
        }
    }
    if (blockIdx.x == 0 && tid < B) a.pos[tid] = s_pos[tid];
    if (blockIdx.x == 0 && tid == 0) *a.steps_done = t;
}

#define DNNHIP_INST(NB, DC) template __global__ void decode_v2<NB, DC>(DecodeArgs);
DNNHIP_INST(1, 1) DNNHIP_INST(1, 2) DNNHIP_INST(1, 3)
DNNHIP_INST(2, 1) DNNHIP_INST(2, 2) DNNHIP_INST(2, 3)
DNNHIP_INST(4, 1) DNNHIP_INST(4, 2) DNNHIP_INST(4, 3)
DNNHIP_INST(8, 1) DNNHIP_INST(8, 2) DNNHIP_INST(8, 3)

const void *decode_kernel_for(int nb, int dc) {
#define DNNHIP_PICK(NB, DC) if (nb == NB && dc == DC) return reinterpret_cast<const void *>(&decode_v2<NB, DC>);
    DNNHIP_PICK(1, 1) DNNHIP_PICK(1, 2) DNNHIP_PICK(1, 3)
    DNNHIP_PICK(2, 1) DNNHIP_PICK(2, 2) DNNHIP_PICK(2, 3)
    DNNHIP_PICK(4, 1) DNNHIP_PICK(4, 2) DNNHIP_PICK(4, 3)
    DNNHIP_PICK(8, 1) DNNHIP_PICK(8, 2) DNNHIP_PICK(8, 3)
    return nullptr;
}

}  // namespace dnnhip
