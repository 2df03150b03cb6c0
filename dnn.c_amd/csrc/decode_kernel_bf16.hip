// decode_kernel_bf16.hip -- the bf16-weight instantiations of the persistent
// decode kernel (1-4 rows; W16A32: the weight matrices are read from the bf16
// copy of the arena and widened to fp32 in registers).  Timing stamps are a
// property of decode_kernel.hip's fp32 instantiations only.
#undef DNNHIP_TRACE
#include "decode_kernel_body.h"

namespace dnnhip {

#define DNNHIP_INST(NB, DC, BF) template __global__ void decode_v3<NB, DC, BF>(DecodeArgs);
DNNHIP_INST(1, 1, true) DNNHIP_INST(1, 2, true) DNNHIP_INST(1, 3, true)
DNNHIP_INST(2, 1, true) DNNHIP_INST(2, 2, true) DNNHIP_INST(2, 3, true)
DNNHIP_INST(4, 1, true) DNNHIP_INST(4, 2, true) DNNHIP_INST(4, 3, true)

}  // namespace dnnhip
