// batch_kernels.hip -- kernels of the batched engine (gfx950, wave64).
//
// One decode step of M rows (or one multi-token prefill) is a chain of
// kernels per layer, the transformer block of the reference
// (transformer_block_forward_cached_ex, transformer.c:211-416) restated for
// many rows at once:
//
//   gemm<EPI_QKV>    rms_norm (norm.c:404-495) -> qkv_proj (nn.c:27-36,
//                    ops_matrix.c:1143-1151) -> split heads (multihead.c:240-263)
//                    -> RoPE (rope.c:20-35) -> Q rows and the K/V cache rows at
//                    each row's position (transformer.c:240-250, kv_cache_append)
//   attn / prefill_attn   scores * 1/sqrt(d_k), causal or prefix-LM mask,
//                    softmax, P.V (transformer.c:256-397)
//   gemm<EPI_RES>    out_proj + bias + residual (ops_elem.c:122-128)
//   gemm<EPI_SWIGLU> rms_norm -> gate/up + biases -> (g/(1+expf(-g)))*u
//                    (nn.c:61-78, simd.h:394-397)
//   gemm<EPI_RES>    down_proj + bias + residual
//
// and per step gemm<EPI_HEAD>: final rms_norm -> tied lm_head + bias
// (gpt.c:117-122, ops_matrix.c:1124-1132) -> argmax, first index of the maximum
// (gpt.c:220-230), whose last workgroup feeds the next step.
//
// GEMM: C[m][n] = sum_k A[m][k] W[n][k] on v_mfma_f32_16x16x4_f32.  Lane l of a
// wavefront holds A[m0 + l%16][k0 + 4(l/16) + j] and W[n0 + l%16][k0 + 4(l/16) + j]
// for j = 0..3 (one 16-byte load each: four MFMAs per 16-column k-step, the
// k values of MFMA j interleaved by 4), and C[m0 + 4(l/16) + v][n0 + l%16] in
// accumulator register v.  The rms_norm is folded in: the k-loop multiplies A
// by gamma and accumulates sum(x^2) from the same registers, and the epilogue
// scales the row by 1/sqrtf(sum(x^2)/d + eps) -- the reference's (x*rs)*gamma
// product reassociated, a rounding-level difference covered by the logit
// tolerance.
//
// Two GEMM shapes: decode (all M <= 64 rows in one tile, 16 columns per
// workgroup, its four wavefronts splitting K; optionally split K over several
// workgroups whose tagged partials the last one to arrive sums in a fixed
// order), and prefill (128 x 128 tiles, a 64 x 64 block per wavefront).

#include "batch.h"
#include <cstdio>
#include <cstdlib>
#include "decode_device.h"

namespace dnnhip {

namespace {

constexpr int NTHR = 256;

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Four consecutive weights of one row as fp32: a 16-byte load (fp32) or an
// 8-byte load of bf16 values widened exactly (bf16 is the top half of fp32).
template <bool BF>
__device__ __forceinline__ f4 ldw4(rsrc_t r, unsigned off_elems) {
    if constexpr (BF) {
        const u2 v = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, off_elems * 2u, 0, CP_NT));
        f4 o;
        o.x = as_float(v.x << 16);
        o.y = as_float(v.x & 0xffff0000u);
        o.z = as_float(v.y << 16);
        o.w = as_float(v.y & 0xffff0000u);
        return o;
    } else {
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off_elems * 4u, 0, CP_NT));
    }
}

__device__ __forceinline__ f4 lda4(rsrc_t r, unsigned off_bytes) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off_bytes, 0, 0));
}

__device__ __forceinline__ void st_pair2(rsrc_t r, size_t pair, float v0, float v1, unsigned tag) {
    const u4 w = {as_uint(v0), tag, as_uint(v1), tag};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, (unsigned)(pair * 8), 0, CP_SC1);
}
__device__ __forceinline__ u4 ld_pair2(rsrc_t r, size_t pair) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)(pair * 8), 0, CP_SC1));
}

// vmcnt(0): this wavefront's loads and stores are complete
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Arrive at a last-arriver counter after this workgroup's stores are complete;
// true in every thread of the workgroup that arrived last (which resets it).
__device__ __forceinline__ bool arrive_last(unsigned *cnt, unsigned n, int *s_flag) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old == n - 1;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = last;
    }
    __syncthreads();
    return *s_flag != 0;
}

// Kernel-entry view of the step state (all workgroups of a launch read the same
// values: only the last workgroup of the head kernel changes them, after every
// other workgroup of that launch has arrived).
__device__ __forceinline__ bool step_done(const StepState *st) {
    return __builtin_nontemporal_load(&st->done) != 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// GEMM.  MT x NT 16x16 tiles per wavefront, WM x WN wavefronts over the block
// tile, KW wavefronts splitting K (WM * WN * KW == 4).  KPW > 0 (decode shape):
// every wavefront owns exactly KPW k-steps and issues all of its loads -- A
// rows first (L2), then its weights (HBM) -- before the first MFMA, so a
// launch keeps its whole weight slice in flight at once.  KPW == 0 (prefill
// shape): a loop over the k-steps, four per iteration.
// DNNHIP_TRACE (timing builds only, never the product): thread 0 of each
// workgroup stamps s_memrealtime at kernel phase boundaries during one chosen
// decode step: trace[kernel slot][workgroup][event].
#ifdef DNNHIP_TRACE
constexpr int BT_SLOTS = 64, BT_WG = 1024, BT_EV = 8;
__device__ unsigned long long g_btrace[BT_SLOTS * BT_WG * BT_EV];
__device__ int g_btrace_step;
#define BTRACE(ST, SLOT, EV)                                                                              \
    do {                                                                                                  \
        if (threadIdx.x == 0 && (ST)->t == g_btrace_step && (SLOT) < BT_SLOTS)                            \
            g_btrace[((size_t)(SLOT) * BT_WG + (blockIdx.x + blockIdx.y * gridDim.x) % BT_WG) * BT_EV + (EV)] = \
                __builtin_amdgcn_s_memrealtime();                                                         \
    } while (0)
#else
#define BTRACE(ST, SLOT, EV) \
    do {                     \
    } while (0)
#endif

template <int MT, int NT, int WM, int WN, int KW, int KPW, bool BF, int EPI, bool NORM, bool AROW = false>
__global__ __launch_bounds__(64 * WM * WN * KW) void gemm_kernel(const GemmArgs g) {
    static_assert(WM * WN * KW == 4 || WM * WN * KW == 8, "four or eight wavefronts");
    constexpr int GT = 64 * WM * WN * KW;                  // threads
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    constexpr int LDR = BN + 1;
    // k-steps per loop iteration (prefill shape; on C4 two beat four by 2.6%
    // and one by 13%)
    constexpr int U = 2;
    __shared__ float red[KW][BM][LDR];
    __shared__ float ssl[KW][BM];
    __shared__ int s_flag;
    __shared__ unsigned s_tag;

    // decode shape: nothing waits on the step state before the main loads are
    // in flight (a launch after the done flag computes and stores nothing)
    constexpr bool DEC = KPW > 0;
    int done_flag = 0;
    if constexpr (!DEC) {
        if (step_done(g.st)) return;
    } else {
        done_flag = __builtin_nontemporal_load(&g.st->done);
    }
    const int tid = threadIdx.x, lane = tid & 63;
    BTRACE(g.st, g.kslot, 0);
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = w % KW, wn = (w / KW) % WN, wm = w / (KW * WN);
    const int tile_n = blockIdx.x / g.ks, ksi = blockIdx.x - tile_n * g.ks, tile_m = blockIdx.y;
    const int r16 = lane & 15, q4 = lane >> 4;
    if (tid == 0) s_tag = __builtin_nontemporal_load(&g.st->tag);

    // this wavefront's k-steps (16 columns each)
    const int nks = g.K / 16, parts = g.ks * KW, part = ksi * KW + kw;
    const int kb0 = part * nks / parts, kb1 = (part + 1) * nks / parts;

    const rsrc_t ra = buf(g.A, (size_t)g.mpad * g.lda * 4);
    const rsrc_t rg = buf(g.gamma, NORM ? (size_t)g.K * 4 : 0);
    unsigned aoff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = tile_m * BM + wm * 16 * MT + 16 * mt + r16;
        int pm = m;
        // a row map only where one is used (a possible load here would make
        // every later wait cover it)
        if (AROW) pm = g.arow[m < g.M ? m : 0];
        aoff[mt] = !g.pk ? (unsigned)(((size_t)pm * g.lda + 4 * q4) * 4)
                   : AROW ? (unsigned)(pk_index(pm, 4 * q4, g.lda) * 4)      // one row's fragment pieces
                          : (unsigned)((((size_t)(tile_m * (BM / 16) + wm * MT + mt) * (g.lda / 16)) * 64 + lane) * 16);
    }
    // bytes between consecutive 16-column k-blocks of A
    const unsigned astep = g.pk ? 1024u : 64u;

    f4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) ss[mt] = 0.f;

    auto kstep = [&](f4 (&a)[MT], const f4 (&b)[NT], const f4 &gm) {
        if (NORM) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                f4 &x = a[mt];
                ss[mt] += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
                x.x *= gm.x; x.y *= gm.y; x.z *= gm.z; x.w *= gm.w;
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                acc[mt][nt] = mfma4(a[mt].x, b[nt].x, acc[mt][nt]);
                acc[mt][nt] = mfma4(a[mt].y, b[nt].y, acc[mt][nt]);
                acc[mt][nt] = mfma4(a[mt].z, b[nt].z, acc[mt][nt]);
                acc[mt][nt] = mfma4(a[mt].w, b[nt].w, acc[mt][nt]);
            }
    };

    // decode shape: the epilogue's operands of this thread's column pairs,
    // loaded before the main loads so that they arrive with them
    constexpr int EP = DEC ? (BM * BN / 2 + GT - 1) / GT : 1;
    float eb0[EP], eb1[EP], er0[EP], er1[EP], ecs[EP], esn[EP];
    int erb[EP], erp[EP];
    if constexpr (DEC) {
#pragma unroll
        for (int e = 0; e < EP; e++) {
            const int i = tid + e * GT;
            const int m = i / (BN / 2), n = 2 * (i - m * (BN / 2));
            const int gm_ = tile_m * BM + m, gn = tile_n * BN + n;
            eb0[e] = eb1[e] = er0[e] = er1[e] = ecs[e] = esn[e] = 0.f;
            erb[e] = erp[e] = 0;
            if (i >= BM * BN / 2 || gm_ >= g.M || gn >= g.N) continue;
            if (EPI == EPI_SWIGLU) { eb0[e] = g.bias[gn >> 1]; eb1[e] = g.bias2[gn >> 1]; }
            else { eb0[e] = g.bias[gn]; eb1[e] = g.bias[gn + 1]; }
            if (EPI == EPI_RES) {
                const size_t ri = g.pk ? pk_index(gm_, gn, g.ldr) : (size_t)gm_ * g.ldr + gn;   // gn even: gn+1 follows
                er0[e] = g.res[ri];
                er1[e] = g.res[ri + 1];
            }
            if (EPI == EPI_QKV) { erb[e] = g.row_b[gm_]; erp[e] = g.row_p[gm_]; }
        }
    }

    if constexpr (KPW > 0) {
        f4 a[KPW][MT], b[KPW][NT], gm[KPW];
#pragma unroll
        for (int u = 0; u < KPW; u++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) a[u][mt] = lda4(ra, aoff[mt] + (unsigned)(kb0 + u) * astep);
            if (NORM) gm[u] = lda4(rg, (unsigned)(((kb0 + u) * 16 + 4 * q4) * 4));
        }
        // weights from the fragment-ordered copy: one contiguous 1 KB (fp32)
        // or 512 B (bf16) per wavefront load (row-major rows gave 16 separate
        // 64-byte pieces per load, about 1 us slower per GEMM at 32 rows)
        const rsrc_t rwp = buf(g.Wp, g.wp_bytes);
        const int nkb = g.ldw / 16;
#pragma unroll
        for (int u = 0; u < KPW; u++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int t16 = tile_n * WN * NT + wn * NT + nt;
                const unsigned po = (unsigned)(((size_t)t16 * nkb + kb0 + u) * 64 + lane) * 4u;
                b[u][nt] = ldw4<BF>(rwp, po);
            }
        // the RoPE loads wait for their positions: issue them only after every
        // main load is in flight (the empty asm keeps the compiler from
        // computing with the rows' positions before this point)
        __builtin_amdgcn_sched_barrier(0);
        if (EPI == EPI_QKV) {
#pragma unroll
            for (int e = 0; e < EP; e++) asm volatile("" : "+v"(erb[e]), "+v"(erp[e]));
        }
        if (EPI == EPI_QKV && g.rope) {
            // RoPE entries of this thread's rows (their positions arrived first)
#pragma unroll
            for (int e = 0; e < EP; e++) {
                const int i = tid + e * GT;
                const int m = i / (BN / 2), n = 2 * (i - m * (BN / 2));
                const int gm_ = tile_m * BM + m, gn = tile_n * BN + n;
                if (i >= BM * BN / 2 || gm_ >= g.M || gn >= 2 * g.D) continue;
                const int d = (gn % g.D) % BK_DK;
                ecs[e] = g.rope[(size_t)erp[e] * (BK_DK / 2) + d / 2];
                esn[e] = g.rope[(size_t)(g.rope_rows + erp[e]) * (BK_DK / 2) + d / 2];
            }
        }
        // keep every load above the first MFMA (the scheduler would otherwise
        // sink loads towards their uses and serialise the HBM round trips)
        __builtin_amdgcn_sched_barrier(0);
#ifdef DNNHIP_TRACE
        __builtin_amdgcn_s_waitcnt(0);                  // timing builds: when every load has landed
        BTRACE(g.st, g.kslot, 5);
#endif
#pragma unroll
        for (int u = 0; u < KPW; u++) kstep(a[u], b[u], gm[u]);
        BTRACE(g.st, g.kslot, 1);
    } else {
        // weights from the fragment-ordered copy: one contiguous 1 KB (fp32)
        // or 512 B (bf16) per wavefront load instead of 16 separate 64-byte
        // pieces of row-major rows (C4 prefill 69 -> 78 TFLOP/s)
        const rsrc_t rwp = buf(g.Wp, g.wp_bytes);
        const int nkb = g.ldw / 16;
        unsigned pb[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int t16 = tile_n * WN * NT + wn * NT + nt;
            pb[nt] = (unsigned)(((size_t)t16 * nkb * 64 + lane) * 4);
        }
        for (int kb = kb0; kb < kb1; kb += U) {
            f4 a[U][MT], b[U][NT], gm[U];
            // every load of the iteration in flight before its first MFMA, in
            // the order of use: the first k-step's (gamma first), then the
            // second's (the scheduler would otherwise sink the second k-step's
            // loads to their uses and wait for each round trip in turn)
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (NORM) gm[u] = lda4(rg, (unsigned)(((kb + u) * 16 + 4 * q4) * 4));
#pragma unroll
                for (int nt = 0; nt < NT; nt++) b[u][nt] = ldw4<BF>(rwp, pb[nt] + (unsigned)((kb + u) * 256));
#pragma unroll
                for (int mt = 0; mt < MT; mt++) a[u][mt] = lda4(ra, aoff[mt] + (unsigned)(kb + u) * astep);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int u = 0; u < U; u++) kstep(a[u], b[u], gm[u]);
        }
    }

    // the wavefront's tiles -> LDS (one copy per K-splitting wavefront)
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int r = wm * 16 * MT + 16 * mt + 4 * q4, c = wn * 16 * NT + 16 * nt + r16;
            red[kw][r + 0][c] = acc[mt][nt].x;
            red[kw][r + 1][c] = acc[mt][nt].y;
            red[kw][r + 2][c] = acc[mt][nt].z;
            red[kw][r + 3][c] = acc[mt][nt].w;
        }
    if (NORM) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            float sv = ss[mt];
            sv += __shfl_xor(sv, 16);
            sv += __shfl_xor(sv, 32);
            if (wn == 0 && q4 == 0) ssl[kw][wm * 16 * MT + 16 * mt + r16] = sv;
        }
    }
    __syncthreads();
    BTRACE(g.st, g.kslot, 2);
    if (DEC && done_flag) return;
    const unsigned tag = s_tag * 128u + (unsigned)g.kslot;

    // split K over workgroups: publish the partial tile (and the rows' partial
    // sums of squares), the last to arrive sums all partials in workgroup
    // order (a fixed order: the result does not depend on which one arrives last)
    const size_t n_main = (size_t)g.ks * g.M * g.N;
    const rsrc_t rp = buf(g.part, g.part ? min(n_main + (size_t)gridDim.x * g.M, g.part_cap) * 8 : 0);
    if (g.ks > 1) {
        for (int i = tid; i < BM * BN / 2; i += GT) {
            const int m = i / (BN / 2), n = 2 * (i - m * (BN / 2));
            const int gm_ = tile_m * BM + m, gn = tile_n * BN + n;
            if (gm_ >= g.M || gn >= g.N) continue;
            float v0 = 0.f, v1 = 0.f;
#pragma unroll
            for (int k = 0; k < KW; k++) { v0 += red[k][m][n]; v1 += red[k][m][n + 1]; }
            st_pair2(rp, ((size_t)ksi * g.M + gm_) * g.N + gn, v0, v1, tag);
        }
        if (NORM)
            for (int m = tid; m < BM; m += GT) {
                const int gm_ = tile_m * BM + m;
                if (gm_ >= g.M) continue;
                float sv = 0.f;
#pragma unroll
                for (int k = 0; k < KW; k++) sv += ssl[k][m];
                put(rp, n_main + ((size_t)tile_n * g.ks + ksi) * g.M + gm_, sv, tag);
            }
        if (!arrive_last(g.cnt + tile_m * (gridDim.x / g.ks) + tile_n, (unsigned)g.ks, &s_flag)) return;
        BTRACE(g.st, g.kslot, 3);
        if (NORM) {
            // the rows' sums of squares over all K, into ssl[0]
            for (int m = tid; m < BM; m += GT) {
                const int gm_ = tile_m * BM + m;
                if (gm_ >= g.M) continue;
                float sv = 0.f;
                for (int k = 0; k < g.ks; k++) {
                    const size_t pr = n_main + ((size_t)tile_n * g.ks + k) * g.M + gm_;
                    u2 p = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rp, (unsigned)(pr * 8), 0, CP_SC1));
                    for (unsigned spin = 0; p.y != tag && spin < SPIN_CAP; spin++) {
                        __builtin_amdgcn_s_sleep(1);
                        p = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rp, (unsigned)(pr * 8), 0, CP_SC1));
                    }
                    sv += as_float(p.x);
                }
                ssl[0][m] = sv;
            }
            __syncthreads();
        }
    }

    // epilogue: two adjacent columns per thread
#pragma unroll
    for (int e = 0; e < (DEC ? EP : 1); e++)
    for (int i = tid + e * GT; i < BM * BN / 2; i += (DEC ? BM * BN : GT)) {
        const int m = i / (BN / 2), n = 2 * (i - m * (BN / 2));
        const int gm_ = tile_m * BM + m, gn = tile_n * BN + n;
        if (gm_ >= g.M || gn >= g.N) continue;
        float v0 = 0.f, v1 = 0.f;
        if (g.ks > 1) {
            // issue every partial's load, then check the tags (re-poll only a
            // partial that is not yet visible)
            constexpr int KSMAX = 8;
            u4 p[KSMAX];
#pragma unroll
            for (int k = 0; k < KSMAX; k++)
                if (k < g.ks) p[k] = ld_pair2(rp, ((size_t)k * g.M + gm_) * g.N + gn);
#pragma unroll
            for (int k = 0; k < KSMAX; k++) {
                if (k >= g.ks) break;
                for (unsigned spin = 0; (p[k].y != tag || p[k].w != tag) && spin < SPIN_CAP; spin++) {
                    __builtin_amdgcn_s_sleep(1);
                    p[k] = ld_pair2(rp, ((size_t)k * g.M + gm_) * g.N + gn);
                }
                v0 += as_float(p[k].x);
                v1 += as_float(p[k].z);
            }
        } else {
#pragma unroll
            for (int k = 0; k < KW; k++) { v0 += red[k][m][n]; v1 += red[k][m][n + 1]; }
        }
        if (NORM) {
            float sv = 0.f;
            if (g.ks > 1) sv = ssl[0][m];
            else {
#pragma unroll
                for (int k = 0; k < KW; k++) sv += ssl[k][m];
            }
            const float rs = 1.0f / sqrtf(sv * (1.0f / (float)g.dnorm) + g.eps);
            v0 *= rs;
            v1 *= rs;
        }
        // the epilogue's operands: prefetched (decode shape) or loaded here
        const bool pf = DEC;
        const int ei = DEC ? e : 0;
        if (EPI == EPI_RES) {
            const float y0 = v0 + (pf ? eb0[ei] : g.bias[gn]), y1 = v1 + (pf ? eb1[ei] : g.bias[gn + 1]);
            const size_t ri = g.pk ? pk_index(gm_, gn, g.ldr) : (size_t)gm_ * g.ldr + gn;
            const float r0 = pf ? er0[ei] : g.res[ri];
            const float r1 = pf ? er1[ei] : g.res[ri + 1];
            float *o = g.out + (g.pk ? pk_index(gm_, gn, g.ldo) : (size_t)gm_ * g.ldo + gn);
            o[0] = r0 + y0;
            o[1] = r1 + y1;
        } else if (EPI == EPI_SWIGLU) {
            // rows 2f (gate) and 2f+1 (up) of the interleaved gate/up matrix
            const int f = gn >> 1;
            const float gt = v0 + (pf ? eb0[ei] : g.bias[f]), up = v1 + (pf ? eb1[ei] : g.bias2[f]);
            g.out[g.pk ? pk_index(gm_, f, g.ldo) : (size_t)gm_ * g.ldo + f] = (gt / (1.0f + expf(-gt))) * up;
        } else if (EPI == EPI_QKV) {
            float y0 = v0 + (pf ? eb0[ei] : g.bias[gn]), y1 = v1 + (pf ? eb1[ei] : g.bias[gn + 1]);
            const int sec = gn / g.D, c = gn - sec * g.D, h = c / BK_DK, d = c - h * BK_DK;
            const int b = pf ? erb[ei] : g.row_b[gm_], p = pf ? erp[ei] : g.row_p[gm_];
            if (sec < 2 && g.rope) {
                const float cs = pf ? ecs[ei] : g.rope[(size_t)p * (BK_DK / 2) + d / 2];
                const float sn = pf ? esn[ei] : g.rope[(size_t)(g.rope_rows + p) * (BK_DK / 2) + d / 2];
                const float e0 = y0, o0 = y1;
                y0 = e0 * cs - o0 * sn;
                y1 = e0 * sn + o0 * cs;
            }
            const size_t head = (((size_t)g.layer * g.B + b) * g.H + h) * (size_t)BK_DK * g.kv_s;
            if (sec == 0) {
                g.q[(size_t)gm_ * g.D + c] = y0;
                g.q[(size_t)gm_ * g.D + c + 1] = y1;
            } else if (sec == 1) {
                g.kc[head + (size_t)d * g.kv_s + p] = y0;
                g.kc[head + (size_t)(d + 1) * g.kv_s + p] = y1;
            } else {
                g.vc[head + (size_t)p * BK_DK + d] = y0;
                g.vc[head + (size_t)p * BK_DK + d + 1] = y1;
            }
        } else {   // EPI_HEAD: logits into the LDS tile for the argmax pass
            const float y0 = v0 + (pf ? eb0[ei] : g.bias[gn]), y1 = v1 + (pf ? eb1[ei] : g.bias[gn + 1]);
            red[0][m][n] = y0;
            red[0][m][n + 1] = y1;
            if (g.logits) {
                const size_t row = g.prefill ? (size_t)gm_ : (size_t)g.st->t * g.M + gm_;
                g.logits[row * g.N + gn] = y0;
                g.logits[row * g.N + gn + 1] = y1;
            }
        }
    }
    if constexpr (EPI == EPI_HEAD) {
        // argmax of this tile's columns per row (first index of the maximum);
        // head_finish_kernel reduces the tiles after this launch
        __syncthreads();
        const int ntn = (g.N + BN - 1) / BN;
        for (int m = tid; m < BM; m += GT) {
            const int gm_ = tile_m * BM + m;
            if (gm_ >= g.M) continue;
            float best = -INFINITY;
            int bi = tile_n * BN;
            for (int n = 0; n < BN; n++) {
                const int gn = tile_n * BN + n;
                if (gn < g.N && red[0][m][n] > best) { best = red[0][m][n]; bi = gn; }
            }
            g.amax[(size_t)gm_ * ntn + tile_n] = make_uint2(as_uint(best), (unsigned)bi);
        }
    }
    BTRACE(g.st, g.kslot, 4);
}

// The lm_head's argmax over its column tiles (gpt.c:220-230: the first index of
// the maximum), then the step's bookkeeping: one workgroup per row.  A row's
// partials, its feed and its state are loaded together up front, the next
// step's embedding row as soon as the token is known; the last workgroup to
// arrive (a counter) advances the step state.  Each row's stop flag reaches it
// as a tagged record, so it needs no fence.
constexpr int FIN_THR = 256;
constexpr int FIN_SLOT = 127;          // tag slot of the stop records (the GEMMs use 0 .. 5 L)
__global__ __launch_bounds__(FIN_THR) void head_finish_kernel(const GemmArgs g) {
    __shared__ float s_bv[FIN_THR / 64];
    __shared__ int s_bi[FIN_THR / 64];
    __shared__ int s_flag;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, m = blockIdx.x;
    BTRACE(g.st, g.kslot + 1, 0);
    const int done = __builtin_nontemporal_load(&g.st->done);
    const bool dec = !g.prefill;
    const int t = dec ? g.st->t : 0;
    const unsigned tag = __builtin_nontemporal_load(&g.st->tag) * 128u + (unsigned)FIN_SLOT;
    const int ntn = g.amax_tiles;
    const int nf = dec ? g.n_feed[m] : 0, ps = dec ? g.pos[m] : 0, rd = dec ? g.row_done[m] : 0;
    const int fnext = (dec && t + 1 < nf) ? g.feed[(size_t)(t + 1) * g.M + m] : -1;
    // the partials in passes of FIN_PASS tiles per thread, every load of a pass
    // issued before the first compare; tiles in increasing order per thread,
    // strict '>' keeps the first maximum
    constexpr int FIN_PASS = 4;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int t0 = 0; t0 < ntn; t0 += FIN_THR * FIN_PASS) {
        uint2 pv[FIN_PASS];
#pragma unroll
        for (int j = 0; j < FIN_PASS; j++) {
            const int tn = t0 + tid + FIN_THR * j;
            pv[j] = tn < ntn ? g.amax[(size_t)m * ntn + tn] : make_uint2(as_uint(-INFINITY), 0x7fffffffu);
        }
#pragma unroll
        for (int j = 0; j < FIN_PASS; j++) {
            const float v = as_float(pv[j].x);
            const int idx = (int)pv[j].y;
            if (v > best || (v == best && idx < bi)) { best = v; bi = idx; }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
    }
    if (lane == 0) { s_bv[w] = best; s_bi[w] = bi; }
    BTRACE(g.st, g.kslot + 1, 2);
    if (done) return;
    __syncthreads();
    best = s_bv[0];
    bi = s_bi[0];
#pragma unroll
    for (int k = 1; k < FIN_THR / 64; k++)
        if (s_bv[k] > best || (s_bv[k] == best && s_bi[k] < bi)) { best = s_bv[k]; bi = s_bi[k]; }
    const int tok = bi == 0x7fffffff ? 0 : bi;
    const rsrc_t rf = buf(g.fin, (size_t)BK_MAXM * 8);
    if (!dec) {
        if (tid == 0) g.ids[m] = tok;
    } else {
        // the next step's embedding row (embedding.c:79-84); the arena's rows
        // are zero past D, as X is
        const int nxt = fnext >= 0 ? fnext : tok;
        const float4 *e = reinterpret_cast<const float4 *>(g.embed + (size_t)nxt * g.ldx);
        for (int c = 4 * tid; c < g.D; c += 4 * FIN_THR)
            *reinterpret_cast<float4 *>(g.x_next + (g.pk ? pk_index(m, c, g.ldx) : (size_t)m * g.ldx + c)) = e[c / 4];
        if (tid == 0) {
            g.ids[(size_t)t * g.M + m] = tok;
            g.pos[m] = ps + 1;
            // rows that stopped in an earlier step stay stopped
            const int dr = rd | (g.eos >= 0 && t >= nf - 1 && tok == g.eos);
            g.row_done[m] = dr;
            put(rf, m, __builtin_bit_cast(float, dr), tag);
        }
    }
    BTRACE(g.st, g.kslot + 1, 4);
    if (!arrive_last(g.head_cnt, gridDim.x, &s_flag)) return;
    BTRACE(g.st, g.kslot + 1, 1);
    if (w == 0) {
        int all = g.eos >= 0;
        if (dec && all)
            for (int b = lane; b < g.M; b += 64) {
                u2 p = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rf, (unsigned)(b * 8), 0, CP_SC1));
                for (unsigned spin = 0; p.y != tag && spin < SPIN_CAP; spin++) {
                    __builtin_amdgcn_s_sleep(1);
                    p = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rf, (unsigned)(b * 8), 0, CP_SC1));
                }
                all &= p.x != 0u;
            }
        all = __all(all);
        if (tid == 0) {
            if (dec) {
                g.st->t = t + 1;
                *g.steps_done = t + 1;
                if (all) g.st->done = 1;
            }
            g.st->tag = g.st->tag + 1;
        }
    }
}

// ---------------------------------------------------------------------------
// Decode attention.  Workgroup (row m, head h, split s) takes the 64-key chunks
// c = s (mod nsplit) of the row's S = pos[m] + 1 cached keys; wavefront w the
// chunks with c / nsplit = w (mod AW).  Lane l holds keys 64c + 4(l%16) + 0..3
// for the scores (dims l/16 + 4i from K^T, summed over the four lane groups),
// and dims 4(l%16) + 0..3 of keys 64c + l/16 + 4i for P.V.  Running max /
// sum per wavefront (transformer.c:354-359), merged across wavefronts in LDS
// and across splits by the last workgroup of the (row, head).
template <int AW>
__global__ __launch_bounds__(64 * AW) void attn_kernel(const AttnArgs a) {
    __shared__ float s_p[AW][64];
    __shared__ float s_o[AW][BK_DK];
    __shared__ float s_ml[AW][2];
    __shared__ int s_flag;
    __shared__ unsigned s_tag;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bh = blockIdx.x / a.nsplit, sp = blockIdx.x - bh * a.nsplit;
    const int m = bh / a.H, h = bh - m * a.H;
    BTRACE(a.st, a.kslot, 0);
    if (tid == 0) s_tag = __builtin_nontemporal_load(&a.st->tag);
    const int r16 = lane & 15, q4 = lane >> 4;
    const size_t head = (((size_t)a.layer * a.B + m) * a.H + h) * (size_t)BK_DK * a.kv_s;
    const rsrc_t rk = buf(a.kc + head, (size_t)BK_DK * a.kv_s * 4);
    const rsrc_t rv = buf(a.vc + head, (size_t)BK_DK * a.kv_s * 4);
    // the step state, the row's length, its query and this wavefront's first
    // chunk of keys and values, all in flight together (the chunk is loaded
    // before the length is known: the descriptor bounds it to the row's cache)
    const int done = __builtin_nontemporal_load(&a.st->done);
    const int posm = a.pos[m];
    float qv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) qv[i] = a.q[(size_t)m * a.D + h * BK_DK + q4 + 4 * i];
    const int c0 = sp + a.nsplit * w;
    // Which wavefronts load their first chunk before the row's length is known:
    // the a.spec leading wavefronts, whose chunk most of the call's rows and
    // steps have (chosen by the host from the positions; with few (row, head)
    // pairs, AW = 8, at least four -- latency matters more there than keys
    // fetched for nothing); the others wait for the length and fetch only
    // chunks that exist.
    const bool spec = w < a.spec;
    f4 kt[16], vv[16];
    auto load_chunk = [&](int c) {
        const int j0 = 64 * c;
#pragma unroll
        for (int i = 0; i < 16; i++)
            kt[i] = lda4(rk, (unsigned)((((size_t)(q4 + 4 * i)) * a.kv_s + j0 + 4 * r16) * 4));
#pragma unroll
        for (int i = 0; i < 16; i++)
            vv[i] = lda4(rv, (unsigned)((((size_t)(j0 + q4 + 4 * i)) * BK_DK + 4 * r16) * 4));
    };
    if (spec) load_chunk(c0);
    __builtin_amdgcn_sched_barrier(0);
    if (done) return;
    const int S = posm + 1;
    const int nch = (S + 63) / 64;

    float mrun = -INFINITY, lrun = 0.f;
    f4 o = {0.f, 0.f, 0.f, 0.f};
    for (int c = c0; c < nch; c += AW * a.nsplit) {
        const int j0 = 64 * c;
        if (c != c0 || !spec) load_chunk(c);
        f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            s.x += qv[i] * kt[i].x; s.y += qv[i] * kt[i].y; s.z += qv[i] * kt[i].z; s.w += qv[i] * kt[i].w;
        }
#pragma unroll
        for (int o2 = 16; o2 <= 32; o2 <<= 1) {
            s.x += __shfl_xor(s.x, o2); s.y += __shfl_xor(s.y, o2);
            s.z += __shfl_xor(s.z, o2); s.w += __shfl_xor(s.w, o2);
        }
        const int jb = j0 + 4 * r16;
        s.x = jb + 0 < S ? s.x * 0.125f : -INFINITY;
        s.y = jb + 1 < S ? s.y * 0.125f : -INFINITY;
        s.z = jb + 2 < S ? s.z * 0.125f : -INFINITY;
        s.w = jb + 3 < S ? s.w * 0.125f : -INFINITY;
        float cm = fmaxf(fmaxf(s.x, s.y), fmaxf(s.z, s.w));
#pragma unroll
        for (int o2 = 1; o2 < 16; o2 <<= 1) cm = fmaxf(cm, __shfl_xor(cm, o2));
        const float mnew = fmaxf(mrun, cm);
        const float sc = expf(mrun - mnew);
        f4 p;
        p.x = expf(s.x - mnew); p.y = expf(s.y - mnew); p.z = expf(s.z - mnew); p.w = expf(s.w - mnew);
        float ps = (p.x + p.y) + (p.z + p.w);
#pragma unroll
        for (int o2 = 1; o2 < 16; o2 <<= 1) ps += __shfl_xor(ps, o2);
        lrun = lrun * sc + ps;
        mrun = mnew;
        if (q4 == 0) *reinterpret_cast<f4 *>(&s_p[w][4 * r16]) = p;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        o.x *= sc; o.y *= sc; o.z *= sc; o.w *= sc;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float pj = s_p[w][q4 + 4 * i];
            o.x += pj * vv[i].x; o.y += pj * vv[i].y; o.z += pj * vv[i].z; o.w += pj * vv[i].w;
        }
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int o2 = 16; o2 <= 32; o2 <<= 1) {
        o.x += __shfl_xor(o.x, o2); o.y += __shfl_xor(o.y, o2);
        o.z += __shfl_xor(o.z, o2); o.w += __shfl_xor(o.w, o2);
    }
    BTRACE(a.st, a.kslot, 1);
    if (q4 == 0) *reinterpret_cast<f4 *>(&s_o[w][4 * r16]) = o;
    if (lane == 0) { s_ml[w][0] = mrun; s_ml[w][1] = lrun; }
    __syncthreads();
    BTRACE(a.st, a.kslot, 2);
    // merge the wavefronts: thread d < 64 owns output dim d
    float om = -INFINITY;
    for (int k = 0; k < AW; k++) om = fmaxf(om, s_ml[k][0]);
    float ol = 0.f, od = 0.f;
    if (tid < BK_DK) {
        for (int k = 0; k < AW; k++) {
            if (s_ml[k][0] == -INFINITY) continue;
            const float f = expf(s_ml[k][0] - om);
            ol += s_ml[k][1] * f;
            od += s_o[k][tid] * f;
        }
    }
    if (a.nsplit == 1) {
        if (tid < BK_DK) {
            const int c = h * BK_DK + tid;
            a.att[a.pk ? pk_index(m, c, a.ldatt) : (size_t)m * a.ldatt + c] = od / ol;
        }
        return;
    }
    // publish (o, m, l) of this split as tagged pairs; the last split of the
    // (row, head) to arrive merges all of them in split order
    const unsigned tag = s_tag * 128u + (unsigned)a.kslot;
    const size_t rec = (size_t)bh * a.nsplit + sp;
    const rsrc_t rp = buf(a.part, (size_t)a.M * a.H * a.nsplit * (BK_DK + 2) * 8);
    if (tid < BK_DK) put(rp, rec * (BK_DK + 2) + tid, od, tag);
    if (tid == 0) { put(rp, rec * (BK_DK + 2) + BK_DK, om, tag); put(rp, rec * (BK_DK + 2) + BK_DK + 1, ol, tag); }
    if (!arrive_last(a.cnt + bh, (unsigned)a.nsplit, &s_flag)) return;
    if (tid >= BK_DK) return;
    // every split's (m, l, o[tid]) loaded at once, tags checked afterwards
    constexpr int NSMAX = 8;
    u2 pm[NSMAX], pl[NSMAX], po[NSMAX];
#pragma unroll
    for (int k = 0; k < NSMAX; k++) {
        if (k >= a.nsplit) break;
        const size_t r = ((size_t)bh * a.nsplit + k) * (BK_DK + 2);
        pm[k] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rp, (unsigned)((r + BK_DK) * 8), 0, CP_SC1));
        pl[k] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rp, (unsigned)((r + BK_DK + 1) * 8), 0, CP_SC1));
        po[k] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rp, (unsigned)((r + tid) * 8), 0, CP_SC1));
    }
    auto settle = [&](u2 &v, size_t pr) {
        for (unsigned spin = 0; v.y != tag && spin < SPIN_CAP; spin++) {
            __builtin_amdgcn_s_sleep(1);
            v = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rp, (unsigned)(pr * 8), 0, CP_SC1));
        }
    };
    float gm = -INFINITY;
#pragma unroll
    for (int k = 0; k < NSMAX; k++) {
        if (k >= a.nsplit) break;
        const size_t r = ((size_t)bh * a.nsplit + k) * (BK_DK + 2);
        settle(pm[k], r + BK_DK);
        settle(pl[k], r + BK_DK + 1);
        settle(po[k], r + tid);
        gm = fmaxf(gm, as_float(pm[k].x));
    }
    float gl = 0.f, gd = 0.f;
#pragma unroll
    for (int k = 0; k < NSMAX; k++) {
        if (k >= a.nsplit) break;
        const float km = as_float(pm[k].x);
        if (km == -INFINITY) continue;
        const float f = expf(km - gm);
        gl += as_float(pl[k].x) * f;
        gd += as_float(po[k].x) * f;
    }
    const int c = h * BK_DK + tid;
    a.att[a.pk ? pk_index(m, c, a.ldatt) : (size_t)m * a.ldatt + c] = gd / gl;
}

// ---------------------------------------------------------------------------
// Prefill attention (the multi-token cached forward, transformer.c:256-397,
// and the full-sequence triangular form, attention.c:259-380).  Workgroup
// (64-row tile of one sequence's new rows, head h), tiles heaviest first;
// wavefront w owns rows 16w .. 16w+15 of the tile.  Per 64-key tile: K^T and
// V staged in LDS (loaded into registers one tile ahead), S = Q K^T on MFMA (A: Q rows from registers, B: K^T from
// LDS), the causal / prefix-LM mask (transformer.c:305-325: a row at
// position p sees keys j < (p < prefix_len ? prefix_len : p + 1) in prefix-LM
// mode, j <= p otherwise), running max / sum per row, P through LDS into the
// A layout, and O += P V on MFMA.
__global__ __launch_bounds__(NTHR) void prefill_attn_kernel(const PrefillAttnArgs a) {
    __shared__ float Ks[BK_DK][65];
    __shared__ float Vs[64][BK_DK + 1];
    __shared__ float Ps[4][16][65];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, q4 = lane >> 4;
    // tile-major: every head of the heaviest tile first (the host orders the tiles)
    const int tile = blockIdx.x / a.H, h = blockIdx.x - tile * a.H;
    const int b = a.tiles[2 * tile], t0 = a.tiles[2 * tile + 1];
    const int nn = a.n_new[b], p0 = a.p0[b], r0 = a.row0[b];
    const int nq = min(64, nn - t0);
    int kv_end = p0 + t0 + nq;
    if (a.mode == 1 && kv_end < a.prefix_len) kv_end = a.prefix_len;
    kv_end = min(kv_end, p0 + nn);
    const size_t head = (((size_t)a.layer * a.B + b) * a.H + h) * (size_t)BK_DK * a.kv_s;
    const rsrc_t rk = buf(a.kc + head, (size_t)BK_DK * a.kv_s * 4);
    const rsrc_t rv = buf(a.vc + head, (size_t)BK_DK * a.kv_s * 4);

    // Q fragments of row 16w + r16 (clamped into the tile), dims 16s + 4 q4 + j
    const int qi = min(16 * w + r16, nq - 1);
    const float *qrow = a.q + (size_t)(r0 + t0 + qi) * a.D + h * BK_DK;
    f4 qf[4];
#pragma unroll
    for (int s = 0; s < 4; s++) qf[s] = *reinterpret_cast<const f4 *>(qrow + 16 * s + 4 * q4);
    // visible keys of the accumulator rows 16w + 4 q4 + v
    int vis[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int p = p0 + t0 + 16 * w + 4 * q4 + v;
        vis[v] = (a.mode == 1 && p < a.prefix_len) ? a.prefix_len : p + 1;
    }
    float mr[4], lr[4];
    f4 O[4];
#pragma unroll
    for (int v = 0; v < 4; v++) { mr[v] = -INFINITY; lr[v] = 0.f; O[v] = f4{0.f, 0.f, 0.f, 0.f}; }

    // this thread's share of a 64-key K^T / V tile, loaded one tile ahead:
    // the next tile's loads are in flight while this one is computed
    f4 kn[4], vn[4];
    auto load_kv = [&](int key0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = tid / 16 + 16 * i, cc = 4 * (tid % 16);
            kn[i] = lda4(rk, (unsigned)(((size_t)rr * a.kv_s + key0 + cc) * 4));
            vn[i] = lda4(rv, (unsigned)(((size_t)(key0 + rr) * BK_DK + cc) * 4));
        }
    };
    if (kv_end > 0) load_kv(0);
    for (int key0 = 0; key0 < kv_end; key0 += 64) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = tid / 16 + 16 * i, cc = 4 * (tid % 16);
            Ks[rr][cc] = kn[i].x; Ks[rr][cc + 1] = kn[i].y; Ks[rr][cc + 2] = kn[i].z; Ks[rr][cc + 3] = kn[i].w;
            Vs[rr][cc] = vn[i].x; Vs[rr][cc + 1] = vn[i].y; Vs[rr][cc + 2] = vn[i].z; Vs[rr][cc + 3] = vn[i].w;
        }
        if (key0 + 64 < kv_end) load_kv(key0 + 64);
        __syncthreads();
        // a wavefront whose 16 rows all lie past the tile's rows (a sequence's
        // last, short tile) has no scores to compute; it still stages its
        // share of K/V, and the next iteration starts at the barrier above
        if (16 * w >= nq) continue;
        f4 S[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) S[nt] = f4{0.f, 0.f, 0.f, 0.f};
        // each 16-dimension group's K^T values read from LDS together, then
        // its MFMAs (read one by one, each read's latency stood before an MFMA)
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float kq[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int nt = 0; nt < 4; nt++) kq[j][nt] = Ks[16 * s + 4 * q4 + j][16 * nt + r16];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int nt = 0; nt < 4; nt++) S[nt] = mfma4(qf[s][j], kq[j][nt], S[nt]);
        }
        float sc[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float mx = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const int key = key0 + 16 * nt + r16;
                const float x = key < vis[v] ? S[nt][v] * 0.125f : -INFINITY;
                S[nt][v] = x;
                mx = fmaxf(mx, x);
            }
#pragma unroll
            for (int o2 = 1; o2 < 16; o2 <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o2));
            const float mnew = fmaxf(mr[v], mx);
            const float base = mnew == -INFINITY ? 0.f : mnew;
            sc[v] = expf(mr[v] - base);
            float ps = 0.f;
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                const float x = expf(S[nt][v] - base);
                S[nt][v] = x;
                ps += x;
            }
#pragma unroll
            for (int o2 = 1; o2 < 16; o2 <<= 1) ps += __shfl_xor(ps, o2);
            lr[v] = lr[v] * sc[v] + ps;
            mr[v] = mnew;
        }
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            Ps[w][4 * q4 + 0][16 * nt + r16] = S[nt].x;
            Ps[w][4 * q4 + 1][16 * nt + r16] = S[nt].y;
            Ps[w][4 * q4 + 2][16 * nt + r16] = S[nt].z;
            Ps[w][4 * q4 + 3][16 * nt + r16] = S[nt].w;
            O[nt].x *= sc[0]; O[nt].y *= sc[1]; O[nt].z *= sc[2]; O[nt].w *= sc[3];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float pq[4], vq[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                pq[j] = Ps[w][r16][16 * s + 4 * q4 + j];
#pragma unroll
                for (int nt = 0; nt < 4; nt++) vq[j][nt] = Vs[16 * s + 4 * q4 + j][16 * nt + r16];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int nt = 0; nt < 4; nt++) O[nt] = mfma4(pq[j], vq[j][nt], O[nt]);
        }
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int i = 16 * w + 4 * q4 + v;
        if (i >= nq) continue;
        const int row = r0 + t0 + i;
        const float inv = lr[v];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int c = h * BK_DK + 16 * nt + r16;
            a.att[a.pk ? pk_index(row, c, a.ldatt) : (size_t)row * a.ldatt + c] = O[nt][v] / inv;
        }
    }
}

// ---------------------------------------------------------------------------
// Embedding rows (embedding.c:79-84) and the reset of the step counters of a
// decode call.
__global__ __launch_bounds__(NTHR) void embed_kernel(const EmbedArgs a) {
    const int m = blockIdx.x;
    if (m == 0 && threadIdx.x == 0 && a.st) { a.st->t = 0; a.st->done = 0; }
    if (threadIdx.x == 0 && a.row_done) a.row_done[m] = 0;
    const int id = a.ids[m];
    if (id < 0 && !a.src) return;
    const float *e = id < 0 ? a.src + (size_t)m * a.ld : a.embed + (size_t)id * a.ld;
    // four columns per thread: one 16-byte piece in either layout (D is a
    // multiple of 64)
    for (int c = 4 * threadIdx.x; c < a.D; c += 4 * NTHR)
        *reinterpret_cast<float4 *>(a.out + (a.pk ? pk_index(m, c, a.ld) : (size_t)m * a.ld + c)) =
            *reinterpret_cast<const float4 *>(e + c);
}

// ---------------------------------------------------------------------------
// rms_norm of rows (norm.c:433-440, 466-471): y = (x * rs) * gamma with
// rs = 1 / sqrtf(sum(x^2) * (1/d) + eps); one workgroup per row.
__global__ __launch_bounds__(NTHR) void rms_rows_kernel(const float *x, const float *gamma, float *y, int d, int ld,
                                                        float eps) {
    __shared__ float s_part[NTHR / 64];
    const int r = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (size_t)r * ld;
    float ss = 0.f;
    for (int c = tid; c < d; c += NTHR) ss += xr[c] * xr[c];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < NTHR / 64; w++) tot += s_part[w];
    const float rs = 1.0f / sqrtf(tot * (1.0f / (float)d) + eps);
    for (int c = tid; c < d; c += NTHR) y[(size_t)r * ld + c] = (xr[c] * rs) * gamma[c];
}

// ---------------------------------------------------------------------------
// launchers

namespace {

// decode shape: all rows in one tile (MT = rows / 16), k-steps per wavefront
// Column tiles of a prefill GEMM: 128, 96 or 64 columns per workgroup.  The
// MFMA-bound prefill GEMMs run a CU's workgroups one after another in effect
// (a launch of 1.05 workgroups per CU costs almost as much as one of 2), so
// the busiest CU's work is its workgroups (rounded up over the device's CUs)
// times their width; the least work wins.  Ties go to 96 columns, then 64:
// narrower tiles put more workgroups on a CU to hide each other's load
// latency, and 96 loads a quarter less per MFMA than 64.  Measured against
// 128 everywhere: 8 x 1024 rows (C4; QKV and out_proj / down at 96, gate/up
// at 64) 78 -> 86 TFLOP/s when introduced; 12,718 rows, K = 512, bf16
// weights (C5; all at 64) 70 -> 74; 1,332 rows (C3) 5.8 -> 4.4 ms.
int prefill_nt(int N, int M) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    const int rows = (M + BK_PBM - 1) / BK_PBM;
    auto cost = [&](int nt) {
        const long long wgs = (long long)((N + 32 * nt - 1) / (32 * nt)) * rows;
        return (wgs + cus - 1) / cus * nt;
    };
    int best = 3;
    if (cost(2) < cost(best)) best = 2;
    if (cost(4) < cost(best)) best = 4;
    return best;
}

// KPW = K / 16 / (4 * ks), chosen by the host among the instantiated values
// (GEMM_KPW_KW8 / GEMM_KPW_KW4 in engine_plan.h list them)
template <int EPI, bool NORM, bool BF, int MT>
hipError_t gemm_decode_mt(const GemmArgs &g, hipStream_t st, int kw, int kpw) {
    const int ntn = (g.N + 15) / 16;
    dim3 grid(ntn * g.ks, (g.M + 16 * MT - 1) / (16 * MT));
#define DNNHIP_KPW(KW, K)                                                                                        \
    case K:                                                                                                      \
        if (EPI == EPI_HEAD && g.arow)                                                                           \
            hipLaunchKernelGGL((gemm_kernel<MT, 1, 1, 1, KW, K, BF, EPI, NORM, EPI == EPI_HEAD>), grid, dim3(64 * KW), 0, st, g); \
        else                                                                                                     \
            hipLaunchKernelGGL((gemm_kernel<MT, 1, 1, 1, KW, K, BF, EPI, NORM>), grid, dim3(64 * KW), 0, st, g); \
        break;
    if (kw == 8) {
        switch (kpw) {
            DNNHIP_KPW(8, 2) DNNHIP_KPW(8, 3) DNNHIP_KPW(8, 4) DNNHIP_KPW(8, 6) DNNHIP_KPW(8, 8)
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (kpw) {
            DNNHIP_KPW(4, 2) DNNHIP_KPW(4, 3) DNNHIP_KPW(4, 4) DNNHIP_KPW(4, 6) DNNHIP_KPW(4, 8) DNNHIP_KPW(4, 12)
            default: return hipErrorInvalidValue;
        }
    }
#undef DNNHIP_KPW
    return hipGetLastError();
}

template <int EPI, bool NORM, bool BF>
hipError_t gemm_decode(const GemmArgs &g, hipStream_t st) {
    const int nks = g.K / 16;
    const int kw = decode_kw(nks, g.ks);
    if (nks % (kw * g.ks)) return hipErrorInvalidValue;
    const int kpw = nks / (kw * g.ks);
    int mt = (g.M + 15) / 16;
    if (g.mt_max > 0 && mt > g.mt_max) mt = g.mt_max;     // row tiles per workgroup (the rest: more workgroups)
    if (g.ks > 1) {
        // the split's partials and last-arriver counters must fit their buffers
        const size_t ntn = (size_t)(g.N + 15) / 16, groups = (size_t)(g.M + 16 * mt - 1) / (16 * mt);
        const size_t need = (size_t)g.ks * g.M * g.N + ntn * g.ks * g.M;
        if (!g.part || need > g.part_cap || groups * ntn > (size_t)g.cnt_cap) return hipErrorInvalidValue;
    }
    switch (mt) {
        case 1: return gemm_decode_mt<EPI, NORM, BF, 1>(g, st, kw, kpw);
        case 2: return gemm_decode_mt<EPI, NORM, BF, 2>(g, st, kw, kpw);
        case 3: return gemm_decode_mt<EPI, NORM, BF, 3>(g, st, kw, kpw);
        case 4: return gemm_decode_mt<EPI, NORM, BF, 4>(g, st, kw, kpw);
        default: return hipErrorInvalidValue;
    }
}

template <int EPI, bool NORM, bool BF>
hipError_t gemm_prefill(const GemmArgs &g, hipStream_t st) {
    // 16-column tiles per wavefront (the workgroup covers 32 * NT columns):
    // DNN_HIP_PREFILL_NT=q,r,s fixes them for the QKV, residual and SwiGLU
    // GEMMs (0: chosen here); read at every launch, as the row-tile overrides
    int req[3] = {0, 0, 0};
    if (const char *e = getenv("DNN_HIP_PREFILL_NT")) sscanf(e, "%d,%d,%d", &req[0], &req[1], &req[2]);
    const int nt = req[EPI] >= 2 && req[EPI] <= 4 ? req[EPI] : prefill_nt(g.N, g.M);
    const int bn = 32 * nt;
    if (g.ks != 1) return hipErrorInvalidValue;          // the prefill shape does not split K
    dim3 grid((g.N + bn - 1) / bn, (g.M + BK_PBM - 1) / BK_PBM);
    if (nt == 2)
        hipLaunchKernelGGL((gemm_kernel<4, 2, 2, 2, 1, 0, BF, EPI, NORM>), grid, dim3(NTHR), 0, st, g);
    else if (nt == 3)
        hipLaunchKernelGGL((gemm_kernel<4, 3, 2, 2, 1, 0, BF, EPI, NORM>), grid, dim3(NTHR), 0, st, g);
    else
        hipLaunchKernelGGL((gemm_kernel<4, 4, 2, 2, 1, 0, BF, EPI, NORM>), grid, dim3(NTHR), 0, st, g);
    return hipGetLastError();
}

template <bool BF>
hipError_t gemm_any(int epi, bool norm, bool prefill, const GemmArgs &g, hipStream_t st) {
    if (prefill) {
        switch (epi) {
            case EPI_QKV: return norm ? gemm_prefill<EPI_QKV, true, BF>(g, st) : hipErrorInvalidValue;
            case EPI_RES: return norm ? hipErrorInvalidValue : gemm_prefill<EPI_RES, false, BF>(g, st);
            case EPI_SWIGLU: return norm ? gemm_prefill<EPI_SWIGLU, true, BF>(g, st) : hipErrorInvalidValue;
            default: return hipErrorInvalidValue;
        }
    }
    switch (epi) {
        case EPI_QKV: return norm ? gemm_decode<EPI_QKV, true, BF>(g, st) : hipErrorInvalidValue;
        case EPI_RES: return norm ? hipErrorInvalidValue : gemm_decode<EPI_RES, false, BF>(g, st);
        case EPI_SWIGLU: return norm ? gemm_decode<EPI_SWIGLU, true, BF>(g, st) : hipErrorInvalidValue;
        case EPI_HEAD: return norm ? gemm_decode<EPI_HEAD, true, BF>(g, st) : gemm_decode<EPI_HEAD, false, BF>(g, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

#ifdef DNNHIP_TRACE
extern "C" int dnn_hip_btrace_arm(int step) {
    static unsigned long long zero[BT_SLOTS * BT_WG * BT_EV];
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_btrace), zero, sizeof zero) != hipSuccess) return -1;
    return hipMemcpyToSymbol(HIP_SYMBOL(g_btrace_step), &step, sizeof step) == hipSuccess ? 0 : -1;
}
extern "C" int dnn_hip_btrace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_btrace), sizeof(unsigned long long) * BT_SLOTS * BT_WG * BT_EV) ==
                   hipSuccess ? 0 : -1;
}
#endif

namespace {
// One thread per (tile, k-block, lane): the lane's 4 elements of the fragment.
template <bool BF>
__global__ __launch_bounds__(256) void pack_kernel(const void *W, void *dst, int N, int ld, size_t total) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int nkb = ld / 16, lane = (int)(i & 63);
    const size_t frag = i >> 6;
    const int tile = (int)(frag / nkb), kb = (int)(frag - (size_t)tile * nkb);
    const int row = tile * 16 + (lane & 15), col = kb * 16 + 4 * (lane >> 4);
    if constexpr (BF) {
        uint2 v = make_uint2(0u, 0u);
        if (row < N) v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(W) + (size_t)row * ld + col);
        reinterpret_cast<uint2 *>(dst)[i] = v;
    } else {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row < N) v = *reinterpret_cast<const float4 *>(static_cast<const float *>(W) + (size_t)row * ld + col);
        reinterpret_cast<float4 *>(dst)[i] = v;
    }
}
}  // namespace

hipError_t launch_pack(const void *W, void *dst, int N, int ld, bool bf16, hipStream_t stream) {
    if (ld % 16) return hipErrorInvalidValue;
    const size_t total = (size_t)((N + 15) / 16) * (ld / 16) * 64;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (bf16)
        hipLaunchKernelGGL(pack_kernel<true>, dim3(blocks), dim3(256), 0, stream, W, dst, N, ld, total);
    else
        hipLaunchKernelGGL(pack_kernel<false>, dim3(blocks), dim3(256), 0, stream, W, dst, N, ld, total);
    return hipGetLastError();
}

hipError_t launch_gemm(int epi, bool norm, bool bf16, bool prefill, const GemmArgs &g, hipStream_t stream) {
    return bf16 ? gemm_any<true>(epi, norm, prefill, g, stream) : gemm_any<false>(epi, norm, prefill, g, stream);
}

hipError_t launch_head_finish(const GemmArgs &g, hipStream_t stream) {
    if (g.M < 1 || g.M > BK_MAXM || !g.fin || !g.head_cnt) return hipErrorInvalidValue;
    hipLaunchKernelGGL(head_finish_kernel, dim3(g.M), dim3(FIN_THR), 0, stream, g);
    return hipGetLastError();
}

hipError_t launch_attn(const AttnArgs &a, hipStream_t stream) {
    // eight wavefronts per (row, head, split) when there are few of them (one
    // workgroup per CU at this register use: every chunk of up to 512 keys in
    // one round), four otherwise (two workgroups per CU)
    if (attn_waves(a.M, a.H) == 8)
        hipLaunchKernelGGL(attn_kernel<8>, dim3(a.M * a.H * a.nsplit), dim3(512), 0, stream, a);
    else
        hipLaunchKernelGGL(attn_kernel<4>, dim3(a.M * a.H * a.nsplit), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill_attn(const PrefillAttnArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(a.n_tiles * a.H), dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_rms_rows(const float *x, const float *gamma, float *y, int n, int d, int ld, float eps,
                           hipStream_t stream) {
    hipLaunchKernelGGL(rms_rows_kernel, dim3(n), dim3(NTHR), 0, stream, x, gamma, y, d, ld, eps);
    return hipGetLastError();
}

hipError_t launch_embed(const EmbedArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(embed_kernel, dim3(a.M), dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

int gemm_tile_rows(bool prefill, int M) { return prefill ? BK_PBM : (M + 15) / 16 * 16; }

}  // namespace dnnhip
