// batch.h -- the batched engine: kernel arguments shared by batch_kernels.hip
// and the C-ABI layer.  Internal: not part of the public headers.
//
// The batched engine runs one decode step (or one multi-token prefill) of M
// rows as a short chain of kernels per layer, replayed from a HIP graph:
//
//   QKV   rms_norm -> fused QKV GEMM + bias -> RoPE -> Q rows, K/V cache rows
//   ATTN  decode: split-S attention over each row's cache; prefill: tiled
//         causal / prefix-LM attention over the new rows and the cache
//   OUT   out_proj GEMM + bias + residual
//   GU    rms_norm -> gate/up GEMM + biases -> SwiGLU
//   DOWN  down GEMM + bias + residual
//
// then HEAD: final rms_norm -> tied lm_head + bias -> argmax (first index of the
// maximum), whose last workgroup also feeds the next step (embedding row of the
// next token, positions, step counters).  The GEMMs run on MFMA
// (v_mfma_f32_16x16x4_f32, fp32 in, fp32 accumulate); the weights are fp32 or
// bf16 (converted to fp32 in registers: W16A32).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "engine_plan.h"

namespace dnnhip {

constexpr int BK_DK = 64;          // head dimension of the attention kernels
constexpr int BK_MAXM = 64;        // rows of the decode GEMM shape (all rows in one tile)
constexpr int BK_PBM = 128;        // prefill GEMM tile rows
constexpr int BK_PBN = 128;        // prefill GEMM tile columns
constexpr int BK_SEQ_ALIGN = 64;   // KV cache row stride is a multiple of this many positions
constexpr int BK_MAXD = 768;       // d_model the engine covers

enum BatchEpi { EPI_QKV = 0, EPI_RES = 1, EPI_SWIGLU = 2, EPI_HEAD = 3 };

// Device-resident state of a session's step loop.  Written only by kernels
// (and the host between calls, while nothing runs).
struct StepState {
    unsigned tag;       // grows by one per launch of a tagged kernel; never reset
    int t;              // steps run in the current decode call
    int done;           // every row has produced eos in its greedy part
    int pad;
};

// C[m][n] = sum_k A[m][k] * W[n][k] (+ epilogue).  A: fp32 rows of lda floats
// (logical row m is physical row arow[m] when arow is set); W: out-major rows of
// ldw elements (fp32 or bf16), zero-padded past the true K, read from its
// fragment-ordered copy Wp.  K (a multiple of 16) counts the padded columns;
// A's padding columns are zero.
struct GemmArgs {
    const float *A;
    const int *arow;
    int lda, M, mpad;           // mpad: rows the A buffer holds (loads past it read 0)
    const void *Wp;             // W in fragment order (fp32 or bf16 elements; see pack_kernel)
    size_t wp_bytes;            // bytes of the packed matrix (loads past it read 0)
    int pk;                     // 1 (decode steps and prefill): A, the residual, the RES / SWIGLU outputs
                                // and the next step's embedding rows are in fragment order (pk_index)
    int ldw, N, K;
    int ks;                     // workgroups per column tile (split K), >= 1
    int mt_max;                 // decode shape: at most this many 16-row tiles per workgroup (0: all rows)
    const float *bias, *bias2;  // [N] (gate/up: bias = gate biases [N/2], bias2 = up biases)
    const float *gamma;         // rms_norm gamma [K] or null
    float eps;
    int dnorm;                  // the true row length of the rms_norm
    // epilogue outputs
    float *out;                 // RES: out[m][n] = res[m][n] + y; SWIGLU: out[m][n/2]; HEAD: logits
    int ldo;
    const float *res;
    int ldr;
    // QKV
    float *q;                   // [M][D]
    float *kc, *vc;             // K^T [L][B][H][DK][S], V [L][B][H][S][DK]
    const int *row_b, *row_p;   // batch row and position of each logical row
    int D, H, kv_s, B, layer;
    const float *rope;          // [2][rope_rows][DK/2] or null
    int rope_rows;
    // split-K partials and last-arriver counters
    uint2 *part;                // [ks][M][N] tagged pairs, then [column tiles][ks][M] row sums of squares
    size_t part_cap;            // pairs the part buffer holds (a launch needing more is refused)
    unsigned *cnt;              // per (row group, column tile)
    int cnt_cap;                // counters at cnt (a launch needing more is refused)
    StepState *st;
    int kslot;                  // distinct per launch of a step: tags are tag * 128 + kslot
    // HEAD
    uint2 *amax;                // [M][column tiles] (value bits, index) per lm_head tile
    unsigned *head_cnt;         // last-arriver counter of head_finish_kernel
    uint2 *fin;                 // [BK_MAXM] tagged stop flags of head_finish_kernel's rows
    int amax_tiles;             // column tiles of the lm_head GEMM (partials per row)
    float *logits;              // [steps][M][V] or null
    int *ids;                   // [steps][M]
    const int *feed, *n_feed;   // [*][M], [M]
    int *pos;                   // [M] cached length per row
    float *x_next;              // residual stream of the next step (embedding rows)
    int ldx;
    const float *embed;         // fp32 embedding [V][ldx]
    int *steps_done;
    int eos, n_steps;
    int *row_done;              // [M]
    int prefill;                // HEAD after a prefill: ids[m], no feed, no step bookkeeping
};

// Decode attention: row m attends to its pos[m] + 1 cached positions.
struct AttnArgs {
    const float *q;             // [M][D]
    float *att;                 // [M][D]
    const float *kc, *vc;
    const int *pos;
    int M, H, kv_s, layer, D, B;
    int ldatt;                  // row stride of att (the out_proj input rows, zero-padded)
    int nsplit;                 // workgroups per (row, head)
    uint2 *part;                // [M*H*nsplit][DK + 2] tagged partials (o[DK], m, l)
    unsigned *cnt;              // [M*H]
    StepState *st;
    int kslot;
    int pk;                     // att rows in fragment order (pk_index)
    int spec;                   // wavefronts w < spec load their first chunk before the row's
                                // length is known
};

// Prefill attention over the new rows of each sequence: logical rows
// [row0[b], row0[b] + n_new[b]) are batch row b at positions
// [p0[b], p0[b] + n_new[b]); mode 0 = causal, 1 = prefix-LM.
struct PrefillAttnArgs {
    const float *q;
    float *att;
    const float *kc, *vc;
    const int *row0, *n_new, *p0;
    const int *tiles;           // [n_tiles][2]: (batch row, first new row of the 64-row tile)
    int n_tiles, H, kv_s, layer, D, B;
    int ldatt;
    int mode, prefix_len;
    StepState *st;
    int pk;                     // att rows in fragment order (pk_index)
};

// Embedding rows: out[m] = embed[ids[m]] (ids: feed row 0 of a decode call, or
// prefill token ids); rows with ids < 0 take row m of src when it is set (an
// embedding input staged row-major), else are left alone.
struct EmbedArgs {
    const float *embed;
    const int *ids;
    float *out;
    const float *src;           // rows with ids < 0: copied from these row-major rows of ld floats (or left alone)
    int M, ld, D;
    int pk;                     // out in fragment order (pk_index)
    StepState *st;              // non-null: reset the step counters of a decode call
    int *row_done;              // non-null: cleared
};

// host-side launchers (batch_kernels.hip); all enqueue on `stream` and return
// a hipError_t.  bf16: W holds bf16 weights.
// Element (m, k) of an activation buffer of row length ld (a multiple of 16)
// in MFMA fragment order: [m/16][k/16][lane = m%16 + 16*((k%16)/4)][k%4], so a
// wavefront's A operand for 16 rows x 16 columns is one contiguous 1 KB piece.
__host__ __device__ inline size_t pk_index(int m, int k, int ld) {
    return ((((size_t)(m >> 4) * (size_t)(ld >> 4) + (size_t)(k >> 4)) << 6) + (size_t)((m & 15) + ((k & 15) >> 2) * 16)) * 4 +
           (size_t)(k & 3);
}

// W (N rows of ld elements, fp32 or bf16) -> dst in fragment order
// [ceil(N/16)][ld/16][64][4], rows past N zero.
hipError_t launch_pack(const void *W, void *dst, int N, int ld, bool bf16, hipStream_t stream);
hipError_t launch_gemm(int epi, bool norm, bool bf16, bool prefill, const GemmArgs &g, hipStream_t stream);
hipError_t launch_head_finish(const GemmArgs &g, hipStream_t stream);
hipError_t launch_attn(const AttnArgs &a, hipStream_t stream);
hipError_t launch_prefill_attn(const PrefillAttnArgs &a, hipStream_t stream);
hipError_t launch_embed(const EmbedArgs &a, hipStream_t stream);
hipError_t launch_rms_rows(const float *x, const float *gamma, float *y, int n, int d, int ld, float eps,
                           hipStream_t stream);
int gemm_tile_rows(bool prefill, int M);

}  // namespace dnnhip
