// decode_kernel.hip -- the persistent gfx950 decode kernel.
//
// One cooperative launch runs n_steps of the GPT token loop of masc-it/dnn.c
// (decoder_lm_generate, gpt.c:306-375) for B rows at once:
//
//   per layer (transformer_block_forward_cached_ex, transformer.c:211-416)
//     A  rms_norm(x) -> qkv GEMV + bias -> RoPE(q,k) -> q buffer, K/V ring write
//     B  split-S decode attention over the row's cached keys, last-arriver combine
//     C  out_proj GEMV + bias + residual (in place on x)
//     D  rms_norm(x) -> gate/up GEMV + bias -> SwiGLU -> act
//     E  down GEMV + bias + residual (in place on x)
//   then
//     F  rms_norm(x) -> tied lm_head GEMV + bias -> per-workgroup argmax
//     G  every workgroup reduces the argmax partials (first index of the max,
//        gpt.c:220-230) and feeds the token to the next step's embedding gather
//
// with one grid barrier after each of A..F.  Nothing returns to the host
// between steps.  Weights are stored out-major (row n of W^T is the K inputs of
// output n, padded to a multiple of 256 floats), so each output is one
// contiguous, coalesced dot product owned by one wavefront: no split-K partials
// to combine.  Activation rows are staged in LDS (RMSNorm applied on the way in)
// and read by every wavefront of the workgroup.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include "decode_kernel.h"

namespace dnnhip {

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

typedef float f4 __attribute__((ext_vector_type(4)));

// Weights are read once per step: stream them past the caches.
__device__ __forceinline__ f4 ld_stream(const float *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
}

// Grid-wide barrier.  Workgroups arrive on one of 8 sub-counters (blockIdx & 7:
// consecutive workgroups are dealt round-robin over the 8 XCDs, so a
// sub-counter collects one XCD's workgroups); the last arrival of a sub-group
// arrives on the top counter, and the last top arrival publishes the barrier's
// generation in a flag the others poll.  Two short chains of same-address
// atomics instead of one long one; polls are relaxed (an acquire load would
// invalidate the XCD's L2 on every poll) and one acquire fence follows.
// Counters and flag are zeroed by the host before each launch.
//
// Every wait is bounded: after SPIN_CAP polls the workgroup sets err[0] and
// goes on, and once err[0] is set every later barrier returns at once, so all
// waves reach the end of the kernel whatever happens; the host discards the
// results of such a launch.
constexpr unsigned SPIN_CAP = 1u << 20;
constexpr int BAR_STRIDE = 32;            // one 256-byte line per counter

__device__ __forceinline__ void grid_sync(unsigned long long *bar, unsigned long long &gen, int *err) {
    gen++;
    __syncthreads();
    if (threadIdx.x == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        const unsigned g = blockIdx.x & 7u;
        const unsigned nsub = (gridDim.x - g + 7u) / 8u;
        const unsigned ngrp = gridDim.x < 8u ? gridDim.x : 8u;
        unsigned long long *sub = bar + g * BAR_STRIDE, *top = bar + 8 * BAR_STRIDE, *flag = bar + 9 * BAR_STRIDE;
        bool published = false;
        if (__hip_atomic_fetch_add(sub, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == gen * nsub - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (__hip_atomic_fetch_add(top, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == gen * ngrp - 1) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                __hip_atomic_store(flag, gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                published = true;
            }
        }
        if (!published) {
            unsigned it = 0;
            while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gen) {
                __builtin_amdgcn_s_sleep(1);
                if (++it == SPIN_CAP) { atomicOr(err, 1); break; }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
}

// Stages rows src[b] (b < nb, n valid floats each) into lds[b][ld], zero-padded
// to ld.  With gamma != nullptr the rows are RMS-normalised on the way in:
// y = (x * rs) * gamma, rs = 1/sqrtf(sum(x^2)/n + eps)   (norm.c:433-440, 466-471).
template <int NB>
__device__ void stage_rows(float *lds, const float *const *src, int nb, int n, int ld,
                           const float *gamma, float eps, float *red) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
    float ss[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) ss[b] = 0.f;
    for (int i = tid; i < ld; i += BLOCK) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float v = (b < nb && i < n) ? src[b][i] : 0.f;
            lds[b * ld + i] = v;
            ss[b] += v * v;
        }
    }
    if (gamma == nullptr) { __syncthreads(); return; }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float t = wave_sum(ss[b]);
        if (lane == 0) red[wid * NB + b] = t;
    }
    __syncthreads();
    float rs[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < WPB; w++) t += red[w * NB + b];
        rs[b] = 1.0f / sqrtf(t * (1.0f / (float)n) + eps);
    }
    for (int i = tid; i < n; i += BLOCK) {
        float g = gamma[i];
#pragma unroll
        for (int b = 0; b < NB; b++) lds[b * ld + i] = (lds[b * ld + i] * rs[b]) * g;
    }
    __syncthreads();
}

// R consecutive out-major weight rows (stride ldw floats) against NB staged
// activation rows; each lane walks float4 columns lane, lane+64, ...; the result
// is wave-reduced so every lane holds acc[r][b].
template <int NB, int R>
__device__ __forceinline__ void dot_rows(const float *__restrict__ w0, int ldw, int nc4,
                                         const float *act, int ld, int lane, float (&acc)[R][NB]) {
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = 0.f;
    for (int c0 = 0; c0 < nc4; c0 += 4 * WAVE) {
        f4 w[4][R];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = c0 + i * WAVE + lane;
            if (c0 + i * WAVE < nc4) {
#pragma unroll
                for (int r = 0; r < R; r++) w[i][r] = ld_stream(w0 + (size_t)r * ldw + 4 * c);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = c0 + i * WAVE + lane;
            if (c0 + i * WAVE < nc4) {
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const f4 a = *reinterpret_cast<const f4 *>(act + b * ld + 4 * c);
#pragma unroll
                    for (int r = 0; r < R; r++)
                        acc[r][b] += w[i][r].x * a.x + w[i][r].y * a.y + w[i][r].z * a.z + w[i][r].w * a.w;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = wave_sum(acc[r][b]);
}

template <int NB>
__global__ void __launch_bounds__(BLOCK)
decode_persistent(DecodeArgs a) {
    // All LDS is one dynamic allocation (lds_bytes()): the small per-workgroup
    // arrays first, then [NB][ldmax] staged activation rows.
    extern __shared__ float smem[];
    float *red = smem;                                  // [WPB*NBMAX]
    float *s_bv = red + WPB * NBMAX;                    // [WPB*NBMAX]
    int *s_bi = reinterpret_cast<int *>(s_bv + WPB * NBMAX);   // [WPB*NBMAX]
    int *s_tok = s_bi + WPB * NBMAX;                    // [MAXB]
    int *s_pos = s_tok + MAXB;                          // [MAXB]
    int *s_done = s_pos + MAXB;                         // [MAXB]
    float *lds = reinterpret_cast<float *>(s_done + MAXB);

    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wid = tid / WAVE;
    const int gwave = blockIdx.x * WPB + wid, nwaves = gridDim.x * WPB;
    const int B = a.B, D = a.D, H = a.H, ldD = a.ldD, ldF = a.ldF;
    const int ncD = ldD / 4, ncF = ldF / 4;
    unsigned long long epoch = 0;

    for (int b = tid; b < B; b += BLOCK) { s_pos[b] = a.pos[b]; s_done[b] = 0; s_tok[b] = 0; }
    __syncthreads();

    int t = 0;
    for (; t < a.n_steps; t++) {
        // tokens of this step: prompt feed, else the previous step's argmax
        for (int b = tid; b < B; b += BLOCK)
            if (t < a.n_feed[b]) s_tok[b] = a.feed[t * B + b];
        __syncthreads();

        int max_s = 0;
        for (int b = 0; b < B; b++) max_s = max(max_s, s_pos[b] + 1);
        const int nch_max = (max_s + CH - 1) / CH;

        for (int l = 0; l < a.L; l++) {
            const LayerW &w = a.layers[l];
            float *kc = a.kc + (size_t)l * B * H * a.max_seq * DK;
            float *vc = a.vc + (size_t)l * B * H * a.max_seq * DK;

            // ---- A: rms_norm -> qkv + bias -> RoPE -> q / K ring / V ring
            for (int b0 = 0; b0 < B; b0 += NB) {
                const int nb = min(NB, B - b0);
                const float *src[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const int bb = b0 + min(b, nb - 1);
                    src[b] = (l == 0) ? a.embed + (size_t)s_tok[bb] * ldD : a.x + (size_t)bb * ldD;
                }
                if (l == 0) {   // embedding gather into the residual stream (embedding.c:79-84)
                    for (int b = 0; b < nb; b++)
                        for (int i = blockIdx.x * BLOCK + tid; i < D; i += gridDim.x * BLOCK)
                            a.x[(size_t)(b0 + b) * ldD + i] = src[b][i];
                }
                stage_rows<NB>(lds, src, nb, D, ldD, w.g_attn, w.eps_attn, red);
                const int nunits = 3 * D / 2;        // RoPE pairs (2k, 2k+1) stay in one wave
                for (int u = gwave; u < nunits; u += nwaves) {
                    const int n = 2 * u;
                    float acc[2][NB];
                    dot_rows<NB, 2>(w.wqkv + (size_t)n * ldD, ldD, ncD, lds, ldD, lane, acc);
                    if (lane < nb) {
                        const int b = lane;
                        float v0 = 0.f, v1 = 0.f;
#pragma unroll
                        for (int bb = 0; bb < NB; bb++)
                            if (bb == b) { v0 = acc[0][bb]; v1 = acc[1][bb]; }
                        v0 = v0 + w.bqkv[n];
                        v1 = v1 + w.bqkv[n + 1];
                        const int sec = n / D, within = n - sec * D;
                        const int h = within / DK, j = within - h * DK;
                        const int row = b0 + b, p = s_pos[row];
                        if (sec < 2 && a.rope_cos) {       // rope.c:28-32
                            const float c = a.rope_cos[(size_t)p * (DK / 2) + j / 2];
                            const float s = a.rope_sin[(size_t)p * (DK / 2) + j / 2];
                            const float e = v0, o = v1;
                            v0 = e * c - o * s;
                            v1 = e * s + o * c;
                        }
                        float *dst;
                        if (sec == 0) dst = a.q + ((size_t)row * H + h) * DK + j;
                        else dst = (sec == 1 ? kc : vc) + (((size_t)row * H + h) * a.max_seq + p) * DK + j;
                        dst[0] = v0;
                        dst[1] = v1;
                    }
                }
                __syncthreads();
            }
            grid_sync(a.bar, epoch, a.err);

            // ---- B: attention of each row's new query over its S = pos+1 cached keys
            {
                const int nunits = B * H * nch_max;
                const float scale = 1.0f / sqrtf((float)DK);
                for (int u = gwave; u < nunits; u += nwaves) {
                    const int c = u % nch_max, bh = u / nch_max;
                    const int b = bh / H, h = bh - b * H;
                    const int S = s_pos[b] + 1, nch = (S + CH - 1) / CH;
                    if (c >= nch) continue;
                    const float *qp = a.q + (size_t)bh * DK;
                    const float *kb = kc + (size_t)bh * a.max_seq * DK;
                    const float *vb = vc + (size_t)bh * a.max_seq * DK;
                    const int j = c * CH + lane;
                    const bool valid = j < S;
                    float s = 0.f;
                    if (valid) {
                        const f4 *k4 = reinterpret_cast<const f4 *>(kb + (size_t)j * DK);
                        const f4 *q4 = reinterpret_cast<const f4 *>(qp);
#pragma unroll
                        for (int d = 0; d < DK / 4; d++) {
                            const f4 kk = k4[d], qq = q4[d];
                            s += qq.x * kk.x + qq.y * kk.y + qq.z * kk.z + qq.w * kk.w;
                        }
                        s = s * scale;
                    }
                    const float m = wave_max(valid ? s : -INFINITY);
                    const float p = valid ? expf(s - m) : 0.f;
                    const float lsum = wave_sum(p);
                    float o = 0.f;
                    const int jn = min(CH, S - c * CH);
                    for (int jj = 0; jj < jn; jj++) {
                        const float pj = __shfl(p, jj, WAVE);
                        o += pj * vb[(size_t)(c * CH + jj) * DK + lane];
                    }
                    float *attrow = a.att + (size_t)b * ldD + h * DK;
                    if (nch == 1) {
                        attrow[lane] = o / lsum;
                        continue;
                    }
                    float *pp = a.part + ((size_t)bh * a.nch_cap + c) * (DK + 2);
                    pp[2 + lane] = o;
                    if (lane == 0) { pp[0] = m; pp[1] = lsum; }
                    __threadfence();
                    unsigned old = 0;
                    if (lane == 0) old = atomicAdd(&a.att_cnt[bh], 1u);
                    old = __shfl(old, 0, WAVE);
                    if (old == (unsigned)(nch - 1)) {       // last chunk in: combine
                        __threadfence();
                        const float *p0 = a.part + (size_t)bh * a.nch_cap * (DK + 2);
                        float M = -INFINITY;
                        for (int cc = 0; cc < nch; cc++) M = fmaxf(M, p0[cc * (DK + 2)]);
                        float Ls = 0.f, O = 0.f;
                        for (int cc = 0; cc < nch; cc++) {
                            const float f = expf(p0[cc * (DK + 2)] - M);
                            Ls += p0[cc * (DK + 2) + 1] * f;
                            O += p0[cc * (DK + 2) + 2 + lane] * f;
                        }
                        attrow[lane] = O / Ls;
                        if (lane == 0) a.att_cnt[bh] = 0u;
                    }
                }
            }
            grid_sync(a.bar, epoch, a.err);

            // ---- C: out_proj + bias + residual
            for (int b0 = 0; b0 < B; b0 += NB) {
                const int nb = min(NB, B - b0);
                const float *src[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) src[b] = a.att + (size_t)(b0 + min(b, nb - 1)) * ldD;
                stage_rows<NB>(lds, src, nb, D, ldD, nullptr, 0.f, red);
                for (int u = gwave; u < D / 2; u += nwaves) {
                    const int n = 2 * u;
                    float acc[2][NB];
                    dot_rows<NB, 2>(w.wo + (size_t)n * ldD, ldD, ncD, lds, ldD, lane, acc);
                    if (lane < nb) {
                        float v0 = 0.f, v1 = 0.f;
#pragma unroll
                        for (int bb = 0; bb < NB; bb++)
                            if (bb == lane) { v0 = acc[0][bb]; v1 = acc[1][bb]; }
                        float *xr = a.x + (size_t)(b0 + lane) * ldD + n;
                        xr[0] = xr[0] + (v0 + w.bo[n]);          // transformer.c:408
                        xr[1] = xr[1] + (v1 + w.bo[n + 1]);
                    }
                }
                __syncthreads();
            }
            grid_sync(a.bar, epoch, a.err);

            // ---- D: rms_norm -> gate/up + bias -> SwiGLU (nn.c:61-78, simd.h:394-397)
            for (int b0 = 0; b0 < B; b0 += NB) {
                const int nb = min(NB, B - b0);
                const float *src[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) src[b] = a.x + (size_t)(b0 + min(b, nb - 1)) * ldD;
                stage_rows<NB>(lds, src, nb, D, ldD, w.g_ffn, w.eps_ffn, red);
                for (int f = gwave; f < a.F; f += nwaves) {
                    float acc[2][NB];
                    dot_rows<NB, 2>(w.wgu + (size_t)f * 2 * ldD, ldD, ncD, lds, ldD, lane, acc);
                    if (lane < nb) {
                        float g = 0.f, up = 0.f;
#pragma unroll
                        for (int bb = 0; bb < NB; bb++)
                            if (bb == lane) { g = acc[0][bb]; up = acc[1][bb]; }
                        g = g + w.bg[f];
                        up = up + w.bu[f];
                        a.act[(size_t)(b0 + lane) * ldF + f] = (g / (1.0f + expf(-g))) * up;
                    }
                }
                __syncthreads();
            }
            grid_sync(a.bar, epoch, a.err);

            // ---- E: down + bias + residual
            for (int b0 = 0; b0 < B; b0 += NB) {
                const int nb = min(NB, B - b0);
                const float *src[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) src[b] = a.act + (size_t)(b0 + min(b, nb - 1)) * ldF;
                stage_rows<NB>(lds, src, nb, a.F, ldF, nullptr, 0.f, red);
                for (int u = gwave; u < D / 2; u += nwaves) {
                    const int n = 2 * u;
                    float acc[2][NB];
                    dot_rows<NB, 2>(w.wd + (size_t)n * ldF, ldF, ncF, lds, ldF, lane, acc);
                    if (lane < nb) {
                        float v0 = 0.f, v1 = 0.f;
#pragma unroll
                        for (int bb = 0; bb < NB; bb++)
                            if (bb == lane) { v0 = acc[0][bb]; v1 = acc[1][bb]; }
                        float *xr = a.x + (size_t)(b0 + lane) * ldD + n;
                        xr[0] = xr[0] + (v0 + w.bd[n]);          // transformer.c:415
                        xr[1] = xr[1] + (v1 + w.bd[n + 1]);
                    }
                }
                __syncthreads();
            }
            grid_sync(a.bar, epoch, a.err);
        }

        // ---- F: final rms_norm -> tied lm_head + bias -> per-workgroup argmax
        for (int b0 = 0; b0 < B; b0 += NB) {
            const int nb = min(NB, B - b0);
            const float *src[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) src[b] = a.x + (size_t)(b0 + min(b, nb - 1)) * ldD;
            stage_rows<NB>(lds, src, nb, D, ldD, a.g_final, a.eps_final, red);
            float bv[NB];
            int bi[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
            for (int u = gwave; u < a.V / 2; u += nwaves) {
                const int v = 2 * u;
                float acc[2][NB];
                dot_rows<NB, 2>(a.embed + (size_t)v * ldD, ldD, ncD, lds, ldD, lane, acc);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const float l0 = acc[0][b] + a.lm_bias[v];
                    const float l1 = acc[1][b] + a.lm_bias[v + 1];
                    if (l0 > bv[b]) { bv[b] = l0; bi[b] = v; }
                    if (l1 > bv[b]) { bv[b] = l1; bi[b] = v + 1; }
                    if (a.logits && lane == 0 && b < nb) {
                        float *lr = a.logits + ((size_t)t * B + b0 + b) * a.V + v;
                        lr[0] = l0;
                        lr[1] = l1;
                    }
                }
            }
            if (lane == 0) {
#pragma unroll
                for (int b = 0; b < NB; b++) { s_bv[wid * NBMAX + b] = bv[b]; s_bi[wid * NBMAX + b] = bi[b]; }
            }
            __syncthreads();
            if (tid < nb) {
                float v = -INFINITY;
                int i = 0x7fffffff;
                for (int ww = 0; ww < WPB; ww++) {
                    const float vv = s_bv[ww * NBMAX + tid];
                    const int ii = s_bi[ww * NBMAX + tid];
                    if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
                }
                a.amax_v[(size_t)(b0 + tid) * gridDim.x + blockIdx.x] = v;
                a.amax_i[(size_t)(b0 + tid) * gridDim.x + blockIdx.x] = i;
            }
            __syncthreads();
        }
        grid_sync(a.bar, epoch, a.err);

        // ---- G: every workgroup reduces the partials -> next token (same in all)
        for (int b = 0; b < B; b++) {
            float v = -INFINITY;
            int i = 0x7fffffff;
            for (int g = tid; g < (int)gridDim.x; g += BLOCK) {
                const float vv = a.amax_v[(size_t)b * gridDim.x + g];
                const int ii = a.amax_i[(size_t)b * gridDim.x + g];
                if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float vv = __shfl_xor(v, o, WAVE);
                const int ii = __shfl_xor(i, o, WAVE);
                if (vv > v || (vv == v && ii < i)) { v = vv; i = ii; }
            }
            if (lane == 0) { s_bv[wid] = v; s_bi[wid] = i; }
            __syncthreads();
            if (tid == 0) {
                for (int ww = 1; ww < WPB; ww++)
                    if (s_bv[ww] > v || (s_bv[ww] == v && s_bi[ww] < i)) { v = s_bv[ww]; i = s_bi[ww]; }
                if (i == 0x7fffffff) i = 0;        // all NaN: argmax keeps index 0
                s_tok[b] = i;
                s_pos[b] += 1;
                if (a.eos >= 0 && t >= a.n_feed[b] - 1 && i == a.eos) s_done[b] = 1;
                if (blockIdx.x == 0) a.ids[(size_t)t * B + b] = i;
            }
            __syncthreads();
        }
        if (a.eos >= 0) {
            int all = 1;
            for (int b = 0; b < B; b++) all &= s_done[b];
            if (all) { t++; break; }
        }
    }
    if (blockIdx.x == 0) {
        for (int b = tid; b < B; b += BLOCK) a.pos[b] = s_pos[b];
        if (tid == 0) *a.steps_done = t;
    }
}

template __global__ void decode_persistent<1>(DecodeArgs);
template __global__ void decode_persistent<2>(DecodeArgs);
template __global__ void decode_persistent<4>(DecodeArgs);
template __global__ void decode_persistent<8>(DecodeArgs);

const void *decode_kernel_for(int nb) {
    switch (nb) {
    case 1: return reinterpret_cast<const void *>(&decode_persistent<1>);
    case 2: return reinterpret_cast<const void *>(&decode_persistent<2>);
    case 4: return reinterpret_cast<const void *>(&decode_persistent<4>);
    default: return reinterpret_cast<const void *>(&decode_persistent<8>);
    }
}

}  // namespace dnnhip
