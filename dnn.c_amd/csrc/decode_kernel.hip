// decode_kernel.hip -- the persistent gfx950 decode kernel.
//
// One launch runs n_steps of the GPT token loop of masc-it/dnn.c
// (decoder_lm_generate, gpt.c:306-375) for B <= 8 rows at once:
//
//   per layer (transformer_block_forward_cached_ex, transformer.c:211-416)
//     A  rms_norm(x) -> qkv GEMV + bias -> RoPE(q, k) -> Q / KN / VN
//     B  attention of one (row, head) per workgroup: each wavefront takes
//        32-key chunks of the S = pos+1 keys with a running max / sum, the
//        workgroup merges the wavefronts' (o, max, sum) in LDS; the wavefront
//        holding position pos appends the new K/V row to the caches
//     C  out_proj GEMV + bias + residual                      -> X1
//     D  rms_norm(X1) -> gate/up GEMV + bias -> SwiGLU        -> ACT
//     E  down GEMV + bias + residual                          -> X2
//   then
//     F  rms_norm(X2) -> tied lm_head GEMV + bias -> argmax partial per workgroup
//     G  one workgroup reduces the partials (first index of the maximum,
//        gpt.c:220-230) and publishes the token, which feeds the next step's
//        embedding rows
//
// Workgroups have roles for the whole launch (A+C, attention, D with a share
// of F, E with a share of F) and each runs its own copy of the step/layer
// loop, so no workgroup runs two consecutive phases: a workgroup stores its
// outputs, then issues the weight loads of its next phase, which land while
// the other roles work (a CU serves its vector-memory requests in order, so
// loads issued between a workgroup's compute and its next wait would delay
// either its stores or that wait).
//
// Synchronisation is dataflow, not grid barriers.  Every value a wavefront
// produces for other workgroups is one 8-byte (value, tag) store with
// device-coherent (sc1) caching; the tag is the global step id.  A workgroup
// that needs a row (the input of a GEMV phase) stages it into LDS once: its 8
// wavefronts split the row, poll their parts until every value carries this
// step's tag, write it to LDS, and meet at a workgroup barrier.  Each
// dependency costs one coherent hop, no L2 writeback/invalidate is issued, and
// the row crosses the fabric once per workgroup rather than once per wavefront.
//
// Weights are out-major (row n = the K inputs of output n, padded to a multiple
// of 256 floats): each output is one contiguous, coalesced dot product owned by
// one wavefront; a workgroup's units of a phase are consecutive, so its outputs
// leave as one block.  Every global access goes through a buffer descriptor
// sized to its tensor, so the hardware range-checks it (out-of-range loads
// read 0, stores are dropped).  This file holds the fp32-weight instantiations
// and the kernel lookup; the body is decode_kernel_body.h.

#include "decode_kernel_body.h"

namespace dnnhip {

#define DNNHIP_INST(NB, DC, BF) template __global__ void decode_v3<NB, DC, BF>(DecodeArgs);
DNNHIP_INST(1, 1, false) DNNHIP_INST(1, 2, false) DNNHIP_INST(1, 3, false)
DNNHIP_INST(2, 1, false) DNNHIP_INST(2, 2, false) DNNHIP_INST(2, 3, false)
DNNHIP_INST(4, 1, false) DNNHIP_INST(4, 2, false) DNNHIP_INST(4, 3, false)
DNNHIP_INST(8, 1, false) DNNHIP_INST(8, 2, false) DNNHIP_INST(8, 3, false)

#ifdef DNNHIP_TRACE
extern "C" int dnn_hip_trace_arm(int step) {
    static unsigned long long zero[256 * TRACE_L * TRACE_E];
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_trace), zero, sizeof zero) != hipSuccess) return -1;
    return hipMemcpyToSymbol(HIP_SYMBOL(g_trace_step), &step, sizeof step) == hipSuccess ? 0 : -1;
}
extern "C" int dnn_hip_trace_read(unsigned long long *out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_trace), sizeof(unsigned long long) * 256 * TRACE_L * TRACE_E) ==
                   hipSuccess ? 0 : -1;
}
#endif

// the bf16-weight instantiations live in decode_kernel_bf16.hip
#define DNNHIP_EXTERN(NB, DC) extern template __global__ void decode_v3<NB, DC, true>(DecodeArgs);
DNNHIP_EXTERN(1, 1) DNNHIP_EXTERN(1, 2) DNNHIP_EXTERN(1, 3)
DNNHIP_EXTERN(2, 1) DNNHIP_EXTERN(2, 2) DNNHIP_EXTERN(2, 3)
DNNHIP_EXTERN(4, 1) DNNHIP_EXTERN(4, 2) DNNHIP_EXTERN(4, 3)

const void *decode_kernel_for(int nb, int dc, bool bf16) {
#define DNNHIP_PICK(NB, DC, BF) \
    if (nb == NB && dc == DC && bf16 == BF) return reinterpret_cast<const void *>(&decode_v3<NB, DC, BF>);
    DNNHIP_PICK(1, 1, false) DNNHIP_PICK(1, 2, false) DNNHIP_PICK(1, 3, false)
    DNNHIP_PICK(2, 1, false) DNNHIP_PICK(2, 2, false) DNNHIP_PICK(2, 3, false)
    DNNHIP_PICK(4, 1, false) DNNHIP_PICK(4, 2, false) DNNHIP_PICK(4, 3, false)
    DNNHIP_PICK(8, 1, false) DNNHIP_PICK(8, 2, false) DNNHIP_PICK(8, 3, false)
    DNNHIP_PICK(1, 1, true) DNNHIP_PICK(1, 2, true) DNNHIP_PICK(1, 3, true)
    DNNHIP_PICK(2, 1, true) DNNHIP_PICK(2, 2, true) DNNHIP_PICK(2, 3, true)
    DNNHIP_PICK(4, 1, true) DNNHIP_PICK(4, 2, true) DNNHIP_PICK(4, 3, true)
    return nullptr;
}

}  // namespace dnnhip
