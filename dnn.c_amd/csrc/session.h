// session.h -- the device model and session objects behind include/dnn_hip.h.
// Internal: shared by the C-ABI layer (dnn_hip.cpp) and the batched engine
// (batch_engine.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/dnn_hip.h"
#include "batch.h"
#include "decode_kernel.h"

struct dnn_hip_model {
    int V, D, L, H, dk, F, ldD, ldF;
    int device;
    int bf16 = 0;                    // weight matrices rounded to bf16 (W16A32)
    char *arena = nullptr;           // fp32 weights, biases, gammas
    uint16_t *arena16 = nullptr;     // bf16 copy of the weight matrices at the same element offsets
    size_t arena_bytes = 0;
    dnnhip::LayerOff *d_layers = nullptr;    // [L] float offsets of each block's tensors
    std::vector<dnnhip::LayerOff> h_layers;
    float eps_final = 1e-5f;
    std::vector<float> eps;          // 2L+1
    float *rope = nullptr;           // [2][rope_rows][dk/2]: cos, then sin
    int rope_rows = 0;
    // byte offsets of every device tensor inside the arena, for the uploads
    struct Off { size_t embed, lm_bias, g_final; std::vector<size_t> l; } off;
    // the weight matrices again in MFMA fragment order for the batched decode
    // GEMMs (built on the device at first use, rebuilt after an update):
    // matrix of N rows and ld columns -> [ceil(N/16)][ld/16][64 lanes][4],
    // lane l holding row 16t + l%16, columns 16kb + 4(l/16) .. +3
    void *packed = nullptr;
    size_t packed_bytes = 0;
    bool packed_valid = false;
    size_t pk_embed = 0;             // element offsets in `packed`
    std::vector<size_t> pk_l;        // [L][4]: wqkv, wo, wgu, wd
};

// Buffers of the batched engine (one per session that uses it).
struct BatchEngine {
    int mcap = 0;                    // rows the activation buffers hold
    int layout = 0;                  // of X, X1, ATT, ACT: 0 row-major (prefill, layer calls), 1 fragment order (decode)
    float *X = nullptr, *X1 = nullptr, *ATT = nullptr, *Q = nullptr, *ACT = nullptr;
    uint2 *part = nullptr;           // split-K partials of the decode GEMMs
    size_t part_pairs = 0;
    uint2 *apart = nullptr;          // split attention partials
    size_t apart_pairs = 0;
    uint2 *amax = nullptr;           // lm_head argmax partials
    size_t amax_pairs = 0;
    unsigned *cnt = nullptr;         // last-arriver counters: [0, CNT_ATT) GEMM tiles, then attention, then head
    dnnhip::StepState *st = nullptr;
    int *row_ident = nullptr;        // [64] 0..63
    int *row_done = nullptr;         // [64]
    int *steps_done = nullptr;
    // prefill inputs
    int *pre_i = nullptr;            // row_b, row_p, pid [mcap] each, then row0, n_new, p0, arow [64], tiles
    size_t pre_cap = 0;
    int *next_ids = nullptr;         // [64]
    float *pre_logits = nullptr;     // [64][V]
    // the captured decode step
    hipGraphExec_t gexec = nullptr;
    const void *gkey[4] = {nullptr, nullptr, nullptr, nullptr};
    int att_spec = 4;                // decode attention: wavefronts that load before the row length is known
    int gspec = -1;                  // att_spec of the captured step graph
    int att_ns = 1;                  // decode attention: workgroups per (row, head)
    int gns = -1;                    // att_ns of the captured step graph
    int geos = -2;
};

struct dnn_hip_session {
    dnn_hip_model *m;
    int B, max_seq;
    int kv_s = 0;                             // KV row stride in positions (max_seq rounded up to 64)
    int batched = 0;                          // decode runs on the batched engine
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    float *kc = nullptr, *vc = nullptr;       // K^T [L][B][H][DK][kv_s], V [L][B][H][kv_s][DK]
    uint2 *xa = nullptr;                      // exchange arena (tagged pairs)
    dnnhip::Exch ex{};
    int *pos = nullptr, *steps_done = nullptr, *err = nullptr;
    int *feed = nullptr, *n_feed = nullptr, *ids = nullptr;
    size_t feed_cap = 0, ids_cap = 0;
    float *logits = nullptr;
    size_t logits_cap = 0;
    int grid_req = 0, grid = 0, grid_cap = 0;
    unsigned next_tag = 1;                    // tags only grow: stale values never match
    int kernel_pref = 0;                      // env DNN_HIP_DECODE_KERNEL: 3 persistent kernel (up to 8 rows) / 6 batched engine
    int kernel_used = 0;                      // 3 or 6: the kernel of the last launch
    int att_splits_req = 0;                   // env DNN_HIP_ATT_SPLITS: workgroups per head in decode_v3 (0 = auto)
    int att_splits = 1;                       // the last decode_v3 launch's
    size_t xa_pairs = 0;
    float last_ms = 0.f;
    // pinned host staging of one call's host-to-device copies (hipHostMalloc):
    // every copy into the device is made from here, never from caller memory
    char *stage = nullptr;
    size_t stage_cap = 0, stage_used = 0;
    std::vector<int> h_pos;
    BatchEngine *eng = nullptr;
};

namespace dnnhip {

// error helpers shared by the C-ABI translation units
int set_error(int code, const char *fmt, ...);

template <class T>
int dalloc(T **p, size_t count) {
    hipError_t e = hipMalloc(reinterpret_cast<void **>(p), (count ? count : 1) * sizeof(T));
    if (e != hipSuccess) {
        *p = nullptr;
        return set_error(DNN_HIP_ENOMEM, "hipMalloc(%zu bytes): %s", count * sizeof(T), hipGetErrorString(e));
    }
    return DNN_HIP_OK;
}

template <class T>
int grow(T **p, size_t *cap, size_t count) {
    if (count <= *cap) return DNN_HIP_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    int rc = dalloc(p, count);
    if (rc == DNN_HIP_OK) *cap = count;
    return rc;
}

// Host-to-device copies of one call go through the session's pinned staging:
// stage_begin reserves `bytes` (rounded up per copy to 256) and resets the
// offset; stage_copy / stage_copy2d copy the caller's bytes into the staging
// buffer and enqueue the asynchronous copy on the session's stream.  Every
// call that stages synchronises its stream before it returns, so the next
// call's staging never overwrites a copy still in flight.
int stage_begin(dnn_hip_session *s, size_t bytes);
int stage_copy(dnn_hip_session *s, void *dst, const void *src, size_t bytes);
int stage_copy2d(dnn_hip_session *s, void *dst, size_t dpitch, const void *src, size_t spitch, size_t width,
                 size_t rows);
inline size_t stage_size(size_t bytes) { return (bytes + 255) / 256 * 256; }

// workgroups per (row, head) of the persistent kernel's attention (dnn_hip.cpp)
int att_splits_for(const dnn_hip_model *m, int B, int ns_cap, int req, int grid, int pmax);
// the static exchange arena of dnn_hip_decode_static on the current device
// (decode_static.hip): its device address is looked up once per device
int static_scratch_setup(int device);

// argument checks of dnn_hip_decode: nf[b] = feed rows of row b
int check_decode(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps,
                 std::vector<int> &nf, int *nf_max);

// batched engine (batch_engine.cpp)
int engine_decode(dnn_hip_session *s, const int *feed, int n_feed_all, const int *n_feed, int n_steps, int eos,
                  int *ids, float *logits, int *steps_done);
int engine_prefill(dnn_hip_session *s, const float *embeds, int n_embed, const int *ids, int n_ids_max,
                   const int *n_ids, int mode, int prefix_len, int *next_ids, float *logits);
int engine_block(dnn_hip_session *s, int layer, const float *x, int n_new, int pos0, int mode, int prefix_len,
                 float *y);
int engine_head(dnn_hip_session *s, const float *x, int n, int norm, float *logits);
int engine_embed(dnn_hip_session *s, const int *ids, int n, float *out);
int engine_rms_norm(dnn_hip_session *s, const float *x, const float *gamma, int n, int d, float eps, float *y);
void engine_destroy(BatchEngine *e);

}  // namespace dnnhip
