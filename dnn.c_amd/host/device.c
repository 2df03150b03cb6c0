/* device.c -- maps each decoder_lm to its HBM mirror (dnn_hip_model).
 *
 * The decoder_lm struct is the reference's and has no room for a device
 * handle, so mirrors live in a small table keyed by the model pointer.  A
 * mirror is refreshed when a fingerprint of the host parameters changes: the
 * parameter pointers and shapes, 4,096 evenly spaced values of every tensor, and
 * the RoPE table pointers.  Training or module_load rewrite whole tensors and
 * change it; decoder_lm_device_sync covers edits the samples could miss. */
#include "device.h"
#include <assert.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAX_MIRRORS 64

typedef struct {
    decoder_lm *lm;
    int weights;            /* DNN_HIP_WEIGHTS_* */
    dnn_hip_model *dm;
    uint64_t print;
} mirror;

static mirror g_mirrors[MAX_MIRRORS];
static int g_device_ready;

void dnn_amd_check(int rc, const char *what) {
    if (rc != DNN_HIP_OK) fprintf(stderr, "dnn_amd: %s failed (%d): %s\n", what, rc, dnn_hip_last_error());
    assert(rc == DNN_HIP_OK && "device call failed");
}

static uint64_t mix(uint64_t h, uint64_t v) {
    h ^= v;
    return h * 1099511628211ULL;
}

/* Identity of the host weights the HBM mirror was made from: every
 * parameter's pointer and size plus 4,096 evenly spaced values of it (about a
 * millisecond for the C2 model).  An in-place edit that touches none of the
 * sampled elements is not seen: such callers call decoder_lm_device_sync, or
 * set DNN_AMD_SYNC=full, which checksums every value (a position-weighted sum,
 * about 80 ms for the C2 model's 365 MB) before each device call. */
static uint64_t fingerprint(decoder_lm *lm) {
    static int full = -1;
    if (full < 0) {
        const char *e = getenv("DNN_AMD_SYNC");
        full = e && strcmp(e, "full") == 0;
    }
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    uint64_t h = 1469598103934665603ULL;
    for (int i = 0; i < n; i++) {
        const long long ne = tensor_numel(ps[i]);
        const float *d = tensor_data_ptr(ps[i]);
        h = mix(h, (uint64_t)(uintptr_t)d);
        h = mix(h, (uint64_t)ne);
        if (full) {
            uint64_t a = 0, b = 0;
            const uint32_t *w = (const uint32_t *)d;
            for (long long k = 0; k < ne; k++) {
                a += w[k];
                b += (uint64_t)w[k] * (uint64_t)(uint32_t)(k + 1);
            }
            h = mix(mix(h, a), b);
        } else {
            const int ns = ne < 4096 ? (int)ne : 4096;
            for (int k = 0; k < ns; k++) {
                uint32_t bits;
                memcpy(&bits, &d[(long long)k * ne / ns], 4);
                h = mix(h, bits);
            }
        }
    }
    tensor *fc = lm->blocks[0]->freqs_cos;
    h = mix(h, (uint64_t)(uintptr_t)fc);
    h = mix(h, fc ? (uint64_t)fc->shape[0] : 0);
    return h;
}

static void params_of(decoder_lm *lm, const float **ptrs, int *n_out, float *eps) {
    int n;
    tensor **ps = module_parameters(&lm->base, &n);
    assert(n == 1 + 12 * lm->n_layers + 2 && "decoder_lm: unexpected parameter count");
    for (int i = 0; i < n; i++) ptrs[i] = tensor_data_ptr(ps[i]);
    for (int l = 0; l < lm->n_layers; l++) {
        eps[2 * l] = lm->blocks[l]->attn_norm->eps;
        eps[2 * l + 1] = lm->blocks[l]->ffn_norm->eps;
    }
    eps[2 * lm->n_layers] = lm->norm->eps;
    *n_out = n;
}

static void upload_rope(decoder_lm *lm, dnn_hip_model *dm) {
    tensor *c = lm->blocks[0]->freqs_cos, *s = lm->blocks[0]->freqs_sin;
    if (c && s) dnn_amd_check(dnn_hip_model_rope(dm, tensor_data_ptr(c), tensor_data_ptr(s), c->shape[0]), "dnn_hip_model_rope");
    else dnn_amd_check(dnn_hip_model_rope(dm, NULL, NULL, 0), "dnn_hip_model_rope");
}

static mirror *find(decoder_lm *lm, int weights) {
    for (int i = 0; i < MAX_MIRRORS; i++)
        if (g_mirrors[i].lm == lm && (lm == NULL || g_mirrors[i].weights == weights)) return &g_mirrors[i];
    return NULL;
}

dnn_hip_model *dnn_amd_device_model(decoder_lm *lm) { return dnn_amd_device_model_ex(lm, DNN_HIP_WEIGHTS_F32); }

dnn_hip_model *dnn_amd_device_model_ex(decoder_lm *lm, int weights) {
    if (!g_device_ready) { dnn_amd_check(dnn_hip_init(0), "dnn_hip_init"); g_device_ready = 1; }
    const int np = 1 + 12 * lm->n_layers + 2;
    const float **ptrs = malloc(sizeof(float *) * (size_t)np);
    float *eps = malloc(sizeof(float) * (size_t)(2 * lm->n_layers + 1));
    int n;
    params_of(lm, ptrs, &n, eps);
    const uint64_t fp = fingerprint(lm);
    mirror *m = find(lm, weights);
    if (!m) {
        m = find(NULL, 0);
        assert(m && "dnn_amd: too many device mirrors; release some with decoder_lm_device_release");
        const transformer_block *b = lm->blocks[0];
        dnn_amd_check(dnn_hip_model_create_ex(lm->vocab_size, lm->d_model, lm->n_layers, b->n_heads, b->d_k,
                                              b->ffn->intermediate_size, ptrs, n, eps, weights, &m->dm),
                      "dnn_hip_model_create_ex");
        m->lm = lm;
        m->weights = weights;
        upload_rope(lm, m->dm);
        m->print = fp;
    } else if (m->print != fp) {
        dnn_amd_check(dnn_hip_model_update(m->dm, ptrs, n), "dnn_hip_model_update");
        upload_rope(lm, m->dm);
        m->print = fp;
    }
    free(ptrs);
    free(eps);
    return m->dm;
}

void decoder_lm_device_sync(decoder_lm *lm) {
    for (int w = DNN_HIP_WEIGHTS_F32; w <= DNN_HIP_WEIGHTS_BF16; w++) {
        mirror *m = find(lm, w);
        if (m) {
            m->print = 0;
            (void)dnn_amd_device_model_ex(lm, w);
        }
    }
    (void)dnn_amd_device_model(lm);
}

void decoder_lm_device_release(decoder_lm *lm) {
    for (int w = DNN_HIP_WEIGHTS_F32; w <= DNN_HIP_WEIGHTS_BF16; w++) {
        mirror *m = find(lm, w);
        if (!m) continue;
        dnn_hip_model_destroy(m->dm);
        m->lm = NULL;
        m->dm = NULL;
    }
}

struct dnn_hip_model *decoder_lm_device_model(decoder_lm *lm) { return dnn_amd_device_model(lm); }

struct dnn_hip_model *decoder_lm_device_model_ex(decoder_lm *lm, int weights) {
    return dnn_amd_device_model_ex(lm, weights);
}
