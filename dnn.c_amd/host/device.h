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
/* Asserts rc == DNN_HIP_OK, printing the device layer's message first. */
void dnn_amd_check(int rc, const char *what);

#endif
