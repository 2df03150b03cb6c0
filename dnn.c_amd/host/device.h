/* device.h -- host-side bridge between a decoder_lm in host pools and its HBM
 * mirror (internal to libdnn_amd). */
#ifndef DNN_AMD_DEVICE_H
#define DNN_AMD_DEVICE_H
#include "dnn/gpt.h"
#include "dnn_hip.h"

/* The device mirror of lm, created or refreshed as needed.  Fatal on failure. */
dnn_hip_model *dnn_amd_device_model(decoder_lm *lm);
/* The same with a choice of weight storage (DNN_HIP_WEIGHTS_*): one mirror per
 * (model, storage). */
dnn_hip_model *dnn_amd_device_model_ex(decoder_lm *lm, int weights);
/* Registry of models built by decoder_lm_create (the block API finds a block's
 * model there). */
void dnn_amd_register_lm(decoder_lm *lm);
/* Device-bound kv caches: whether c is bound, and a copy of its device rows
 * into its host tensors. */
int dnn_amd_cache_is_bound(kv_cache *c);
void dnn_amd_cache_sync(kv_cache *c);
/* Asserts rc == DNN_HIP_OK, printing the device layer's message first. */
void dnn_amd_check(int rc, const char *what);

#endif
