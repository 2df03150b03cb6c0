// decode_device.h -- device helpers shared by the decode kernels: buffer
// descriptors and cache policies, tagged exchange values and their bounded
// waits, LDS staging of tagged rows, GEMV building blocks.
#pragma once
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
// voff: per-lane byte offset (VGPR); soff: wave-uniform byte offset (SGPR), so
// unrolled loads that differ by a uniform stride share one address register
template <int CP>
__device__ __forceinline__ float ld1s(rsrc_t r, unsigned voff, unsigned soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, (int)soff, CP));
}
__device__ __forceinline__ void st1(rsrc_t r, size_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (unsigned)off, 0, CP_SC1);
}
__device__ __forceinline__ void put(rsrc_t xa, size_t pair, float v, unsigned tag) {
    u2 w = {__builtin_bit_cast(unsigned, v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(w, xa, (unsigned)(pair * 8), 0, CP_SC1);
}

// Wavefront reductions with DPP row operations (a few ALU cycles per step;
// __shfl_xor costs an LDS permute and a wait per step): pairs, quads, half
// rows, rows, then rows 0+1 into row 1 and rows 0..3 into row 3; lane 63
// holds the total, broadcast with readlane.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp(float v, float fill) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill), __builtin_bit_cast(int, v),
                                                                 CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xb1, 0xf>(v, 0.f);      // quad_perm [1,0,3,2]
    v += dpp<0x4e, 0xf>(v, 0.f);      // quad_perm [2,3,0,1]
    v += dpp<0x141, 0xf>(v, 0.f);     // row_half_mirror
    v += dpp<0x140, 0xf>(v, 0.f);     // row_mirror
    v += dpp<0x142, 0xa>(v, 0.f);     // row_bcast:15 into rows 1, 3
    v += dpp<0x143, 0xc>(v, 0.f);     // row_bcast:31 into rows 2, 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xb1, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp<0x4e, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp<0x141, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp<0x140, 0xf>(v, -INFINITY));
    v = fmaxf(v, dpp<0x142, 0xa>(v, -INFINITY));
    v = fmaxf(v, dpp<0x143, 0xc>(v, -INFINITY));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float bcast(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Workgroup barrier for hand-offs through LDS only: waits for this wavefront's
// LDS operations, not for its vector-memory ones (__syncthreads' fence also
// drains vmcnt), so weight loads issued for a later phase stay in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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

// A single tagged value per lane at pair index `p` (p < 0: nothing to wait for).
__device__ __forceinline__ float poll1(rsrc_t xa, long p, unsigned tag, Waiter &w) {
    w.reset();
    for (;;) {
        u2 q = {0u, tag};
        if (p >= 0) q = __builtin_amdgcn_raw_buffer_load_b64(xa, (unsigned)(p * 8), 0, CP_SC1);
        if (__all(q.y == tag) || !w.again()) return as_float(q.x);
    }
}

// Stage nrows tagged rows (n valid values each, row r at pair index
// base0 + r * stride) into LDS rows of stride ld.  The rows are cut into
// 128-value chunks (64 lanes x 2 pairs); chunk c goes to wavefront c % WPB.
// Columns >= n are left alone (zeroed once at launch).
template <int NCMAX>
__device__ __forceinline__ void stage_rows(float *dst, int ld, int n, int nrows, size_t base0, size_t stride,
                                           rsrc_t xa, unsigned tag, int wid, int lane, Waiter &wt) {
    const int cpr = (n + 127) / 128, total = nrows * cpr;
    u4 q[NCMAX];
    wt.reset();
    for (;;) {
        bool ok = true;
        // branch-free: chunks past the end re-read the last one, so every load
        // of the poll is issued before the first wait
#pragma unroll
        for (int i = 0; i < NCMAX; i++) {
            const int c = min(wid + i * WPB, total - 1);
            const int r = c / cpr, col = (c - r * cpr) * 128 + 2 * lane;
            q[i] = __builtin_amdgcn_raw_buffer_load_b128(xa, (unsigned)((base0 + r * stride + col) * 8), 0, CP_SC1);
            const unsigned t0 = q[i].y, t1 = q[i].w;
            ok &= (col >= n || t0 == tag) && (col + 1 >= n || t1 == tag);
        }
        if (__all(ok) || !wt.again()) break;
    }
#pragma unroll
    for (int i = 0; i < NCMAX; i++) {
        const int c = wid + i * WPB;
        if (c < total) {
            const int r = c / cpr, col = (c - r * cpr) * 128 + 2 * lane;
            if (col < n) dst[r * ld + col] = as_float(q[i].x);
            if (col + 1 < n) dst[r * ld + col + 1] = as_float(q[i].z);
        }
    }
}

// Reciprocal RMS of nb LDS rows (norm.c:433-440): rs = 1/sqrtf(sum(x^2) * (1/n) + eps).
template <int NB, int DC>
__device__ __forceinline__ void rms_lds(const float *xs, int ld, int n, float eps, int lane, float (&rs)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < DC; k++) {
            const f4 x = *reinterpret_cast<const f4 *>(xs + b * ld + k * 256 + 4 * lane);
            ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
        }
        rs[b] = 1.0f / sqrtf(wave_sum(ss) * (1.0f / (float)n) + eps);
    }
}

// One lane's piece of a weight row chunk: 4 consecutive weights, fp32 (f4) or
// bf16 (u2, element 0 in the low half of .x), widened to fp32 where used.
template <bool BF> struct WPiece { typedef f4 T; };
template <> struct WPiece<true> { typedef u2 T; };
__device__ __forceinline__ f4 widen(f4 v) { return v; }
__device__ __forceinline__ f4 widen(u2 v) {
    f4 r;
    r.x = as_float(v.x << 16); r.y = as_float(v.x & 0xffff0000u);
    r.z = as_float(v.y << 16); r.w = as_float(v.y & 0xffff0000u);
    return r;
}
// lane `lane`'s piece of the 256-column chunk starting at element `off`
template <bool BF>
__device__ __forceinline__ typename WPiece<BF>::T ld_piece(rsrc_t rm, size_t off, int lane) {
    if constexpr (BF)
        return __builtin_amdgcn_raw_buffer_load_b64(rm, (unsigned)((off + 4 * lane) * 2), 0, CP_NT);
    else
        return ld4<CP_NT>(rm, (off + 4 * lane) * 4);
}

// weights of R consecutive out-major rows starting at element `off` of the
// matrix arena `rm` (fp32, or bf16 at the same element offsets; row stride ld
// elements), DC chunks of 256 columns each
template <int R, int DC, bool BF>
__device__ __forceinline__ void load_rows(typename WPiece<BF>::T (&w)[R][DC], rsrc_t rm, size_t off, int ld, int lane) {
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int k = 0; k < DC; k++) w[r][k] = ld_piece<BF>(rm, off + (size_t)r * ld + k * 256, lane);
}

// Per-lane partial sums of the row dot products, before the wavefront
// reduction: s[r * NB + b] = this lane's share of w[r] . y_b, y_b = LDS row b,
// optionally normalised as (x * rs) * gamma (norm.c:466-471) first.
template <int R, int NB, int DC, bool NORM, typename WT>
__device__ __forceinline__ void part_lds(const WT (&w)[R][DC], const float *xs, int ld, const float (&rs)[NB],
                                         const f4 (&g)[DC], int lane, float *s) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
        for (int r = 0; r < R; r++) s[r * NB + b] = 0.f;
#pragma unroll
        for (int k = 0; k < DC; k++) {
            f4 y = *reinterpret_cast<const f4 *>(xs + b * ld + k * 256 + 4 * lane);
            if (NORM) {
                y.x = (y.x * rs[b]) * g[k].x; y.y = (y.y * rs[b]) * g[k].y;
                y.z = (y.z * rs[b]) * g[k].z; y.w = (y.w * rs[b]) * g[k].w;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const f4 wv = widen(w[r][k]);
                s[r * NB + b] += wv.x * y.x + wv.y * y.y + wv.z * y.z + wv.w * y.w;
            }
        }
    }
}

// N independent wave sums with their DPP steps interleaved (no hazard wait
// states between dependent steps); each value gets the same additions in the
// same order as wave_sum.
template <int N>
__device__ __forceinline__ void wave_sum_n(float *v) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0xb1, 0xf>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x4e, 0xf>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x141, 0xf>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x140, 0xf>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x142, 0xa>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x143, 0xc>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[i]), 63));
}

// R weight rows of one work unit and their biases (fp32 arena), loaded
// together ahead of the unit's phase.
template <int R, int DC, bool BF = false>
struct RowUnit {
    typename WPiece<BF>::T w[R][DC];
    float bias[R];
};
template <int R, int DC, bool BF>
__device__ __forceinline__ void load_unit(RowUnit<R, DC, BF> &u, rsrc_t rw, rsrc_t rm, size_t woff, int ld,
                                          const size_t (&boff)[R], int lane) {
    load_rows<R, DC, BF>(u.w, rm, woff, ld, lane);
#pragma unroll
    for (int r = 0; r < R; r++) u.bias[r] = ld1<0>(rw, boff[r] * 4);
}

// Output block of one GEMV round of a workgroup: its NU wavefronts own the
// consecutive units u0 .. u0+NU-1, R outputs each, for NB batch rows, and
// left them in LDS (out[w][b*R + r]).  One wavefront writes them as tagged
// pairs; consecutive lanes hit consecutive pairs, so every row's block leaves
// as one coalesced store instead of WPB*R scattered 8-byte ones (scattered
// single-value stores to shared lines made each hop several times slower).
template <int R, int NB, int NU = WPB>
__device__ __forceinline__ void write_block(const float *out, rsrc_t xa, size_t row0, size_t rstride, int u0, int nu,
                                            int B, unsigned tag, int lane) {
    constexpr int PER = NU * R;
#pragma unroll
    for (int i0 = 0; i0 < NB * PER; i0 += WAVE) {
        const int i = i0 + lane;
        const int b = i / PER, j = i - b * PER, w = j / R, r = j - w * R;
        if (i < NB * PER && b < B && u0 + w < nu)
            put(xa, row0 + b * rstride + (size_t)(u0 + w) * R + r, out[w * NB * R + b * R + r], tag);
    }
}

// The layer's offsets as wave-uniform (SGPR) values: loaded once per wave and
// broadcast, so every address derived from them stays scalar.
__device__ __forceinline__ LayerOff load_layer(const LayerOff *p) {
    LayerOff w = *p;
    auto u = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
    auto f = [](float v) { return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v))); };
    w.wqkv = u(w.wqkv); w.bqkv = u(w.bqkv); w.wo = u(w.wo); w.bo = u(w.bo);
    w.g_attn = u(w.g_attn); w.g_ffn = u(w.g_ffn); w.wgu = u(w.wgu); w.bg = u(w.bg);
    w.bu = u(w.bu); w.wd = u(w.wd); w.bd = u(w.bd);
    w.eps_attn = f(w.eps_attn); w.eps_ffn = f(w.eps_ffn);
    return w;
}

template <int DC>
__device__ __forceinline__ void load_gamma(f4 (&g)[DC], rsrc_t rw, size_t off, int lane) {
#pragma unroll
    for (int k = 0; k < DC; k++) g[k] = ld4<0>(rw, (off + k * 256 + 4 * lane) * 4);
}

}  // namespace dnnhip
