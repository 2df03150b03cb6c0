/* multihead.h -- head split / merge layout transforms (reference
 * include/multihead.h:20-33), on the device.  Outputs are new contiguous
 * scratch tensors.  Forward only. */
#ifndef DNN_MULTIHEAD_H
#define DNN_MULTIHEAD_H
#include "tensor.h"

/* [B, N, H * d_k] -> [B, H, N, d_k] (contiguous input). */
tensor *tensor_split_heads(struct mem_pool *scratch, tensor *t, int H);
/* [B, H, N, d_k] -> [B, N, H * d_k]; reads t's elements in storage order from
 * its offset, as the reference does (multihead.c:199-212). */
tensor *tensor_merge_heads(struct mem_pool *scratch, tensor *t);
/* Fused QKV projection output [B, N, 3 * H * d_k] (contiguous) -> Q, K, V, each
 * [B, H, N, d_k]: columns [0, H*d_k) are Q, then K, then V (multihead.c:300-348). */
void tensor_split_qkv_heads(struct mem_pool *scratch,
                            tensor *qkv, int H,
                            tensor **Qh_out, tensor **Kh_out, tensor **Vh_out);

#endif
