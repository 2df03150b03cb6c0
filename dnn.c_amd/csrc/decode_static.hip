// decode_static.hip -- dnn_hip_decode_static: the persistent decode kernel
// (decode_v3) on buffers the caller owns, with its scratch -- the exchange
// arena of tagged values and two status words -- in a file-scope device array
// instead of session allocations.  The call allocates nothing and does not
// synchronise the host, so callers that cannot allocate (HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc) can use it.
//
// Each GPU holds its own copy of the array until the process ends; its device
// address is looked up once per device (static_scratch_setup, from
// dnn_hip_init or the first call on a device) and only that address is handed
// to kernels.  Every call on a GPU shares the array: calls that overlap on one
// GPU race.  Stale contents are harmless: every value carries the step tag it
// was written at and tags only grow (one counter per device), and the status
// words are cleared by a kernel at the start of each call.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdlib>
#include <mutex>

#include "../../include/dnn_hip.h"
#include "decode_kernel.h"
#include "session.h"

using namespace dnnhip;

namespace {
constexpr size_t STATIC_HEAD = 256;                            // bytes of status words before the arena
constexpr size_t STATIC_XA_PAIRS = DNN_HIP_STATIC_EXCHANGE_PAIRS;   // 8 MiB of (value, tag) pairs
constexpr int MAX_DEV = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[STATIC_HEAD + STATIC_XA_PAIRS * 8];

namespace {

std::mutex g_mu;
unsigned char *g_ptr[MAX_DEV];      // the array's device address on each GPU
unsigned g_tag[MAX_DEV];            // next step tag on each GPU (tag 0: never a step's)

// status words: [0] error bits of the last call, [1] steps it ran
__global__ void status_clear_kernel(int *st) {
    if (threadIdx.x < 2) st[threadIdx.x] = 0;
}

}  // namespace

int dnnhip::static_scratch_setup(int device) {
    if (device < 0 || device >= MAX_DEV) return set_error(DNN_HIP_EINVAL, "device %d: at most %d", device, MAX_DEV);
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return DNN_HIP_OK;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess || cur != device)
        return set_error(DNN_HIP_EDEVICE, "static scratch: device %d is not current (%d)", device, cur);
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_error(DNN_HIP_EDEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_ptr[device] = static_cast<unsigned char *>(p);
    g_tag[device] = 1;
    return DNN_HIP_OK;
}

extern "C" {

size_t dnn_hip_kv_floats(const dnn_hip_model *m, int batch, int max_seq) {
    if (!m || batch < 1 || max_seq < 1) return 0;
    const size_t kv_s = ((size_t)max_seq + 63) / 64 * 64;
    return (size_t)m->L * batch * m->H * kv_s * DK + (size_t)CH * DK;
}

int dnn_hip_decode_static(dnn_hip_model *m, int batch, int max_seq, float *kc, float *vc, int *pos, const int *feed,
                          const int *n_feed, int n_steps, int eos, int max_len, int *ids, float *logits,
                          void *stream) {
    if (!m || !kc || !vc || !pos || !feed || !n_feed || !ids) return set_error(DNN_HIP_EINVAL, "NULL argument");
    if (batch < 1 || batch > MAXB) return set_error(DNN_HIP_EINVAL, "batch %d outside [1,%d]", batch, MAXB);
    if (m->bf16) return set_error(DNN_HIP_EINVAL, "dnn_hip_decode_static runs fp32-weight models");
    if (max_seq < 1 || n_steps < 1) return set_error(DNN_HIP_EINVAL, "max_seq %d / n_steps %d", max_seq, n_steps);
    if (max_len < n_steps || max_len > max_seq || (m->rope && max_len > m->rope_rows))
        return set_error(DNN_HIP_ERANGE, "max_len %d: needs n_steps %d <= max_len <= max_seq %d (and the RoPE rows %d)",
                         max_len, n_steps, max_seq, m->rope ? m->rope_rows : max_seq);
    int dev = 0, n_cu = 0, lds_max = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev != m->device)
        return set_error(DNN_HIP_EINVAL, "the model lives on device %d, device %d is current", m->device, dev);
    int rc = static_scratch_setup(dev);
    if (rc) return rc;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0) n_cu = 256;
    if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return set_error(DNN_HIP_EDEVICE, "device attributes");
    Exch ex{m->ldD, m->ldF, m->D, batch, n_cu, m->H, batch * m->H <= ATT_SPLIT_HEADS ? ATT_SPLIT_MAX : 1};
    if (ex.total(m->L) > STATIC_XA_PAIRS)
        return set_error(DNN_HIP_EINVAL, "this model and batch need %zu exchange pairs; the static arena holds %zu",
                         ex.total(m->L), STATIC_XA_PAIRS);
    const size_t kv_bytes = dnn_hip_kv_floats(m, batch, max_seq) * sizeof(float);
    if (kv_bytes >= 0x7fffffffu) return set_error(DNN_HIP_EINVAL, "KV cache of %zu bytes: must stay < 2 GiB", kv_bytes);
    const int nb = batch > 4 ? 8 : batch > 2 ? 4 : batch > 1 ? 2 : 1;
    const void *kern = decode_kernel_for(nb, m->ldD / LDALIGN, false);
    const size_t shmem = lds_bytes(nb, m->ldD, m->ldF);
    if (!kern || shmem > (size_t)lds_max) return set_error(DNN_HIP_EINVAL, "no decode kernel for this shape");
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem) != hipSuccess)
        return set_error(DNN_HIP_EDEVICE, "decode kernel attributes");

    unsigned char *base = g_ptr[dev];
    int *status = reinterpret_cast<int *>(base);
    DecodeArgs a{};
    a.V = m->V; a.D = m->D; a.L = m->L; a.H = m->H; a.F = m->F; a.ldD = m->ldD; a.ldF = m->ldF;
    a.wts = reinterpret_cast<const float *>(m->arena);
    a.wts_bytes = (uint32_t)m->arena_bytes;
    a.embed = (uint32_t)(m->off.embed / sizeof(float));
    a.lm_bias = (uint32_t)(m->off.lm_bias / sizeof(float));
    a.g_final = (uint32_t)(m->off.g_final / sizeof(float));
    a.layers = m->d_layers;
    a.eps_final = m->eps_final;
    a.rope = m->rope; a.rope_rows = m->rope_rows;
    a.B = batch; a.max_seq = (int)(((size_t)max_seq + 63) / 64 * 64);
    a.kc = kc; a.vc = vc;
    a.xa = reinterpret_cast<uint2 *>(base + STATIC_HEAD);
    a.ex = ex;
    a.ex.ns = att_splits_for(m, batch, ex.ns, 0, n_cu, max_len);
    a.pos = pos; a.feed = feed; a.n_feed = n_feed; a.ids = ids; a.logits = logits;
    a.n_steps = n_steps; a.eos = eos;
    a.err = status; a.steps_done = status + 1;
    a.seq_limit = max_len;
    Roles roles{};
    if (!plan_roles(n_cu, m->D, m->F, m->ldD, m->ldF, batch * m->H * a.ex.ns, roles, hold_rounds(nb, m->ldD / LDALIGN)))
        return set_error(DNN_HIP_EINVAL, "a grid of %d workgroups is too small for the decode kernel's roles", n_cu);
    a.n_ac = roles.n_ac; a.n_d = roles.n_d; a.n_e = roles.n_e;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        a.step0 = g_tag[dev];
        g_tag[dev] += (unsigned)n_steps;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(status_clear_kernel, dim3(1), dim3(64), 0, st, status);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(DNN_HIP_EDEVICE, "status clear: %s", hipGetErrorString(e));
    void *kargs[] = {&a};
    e = hipLaunchKernel(kern, dim3(n_cu), dim3(BLOCK), kargs, shmem, st);
    if (e != hipSuccess) return set_error(DNN_HIP_EDEVICE, "decode launch: %s", hipGetErrorString(e));
    return DNN_HIP_OK;
}

int dnn_hip_decode_static_status(void *stream, int *steps_done, int *err_bits) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(DNN_HIP_EDEVICE, "hipGetDevice");
    int rc = static_scratch_setup(dev);
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    int st[2] = {0, 0};
    if (e == hipSuccess) e = hipMemcpy(st, g_ptr[dev], sizeof st, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error(DNN_HIP_EDEVICE, "static decode status: %s", hipGetErrorString(e));
    if (steps_done) *steps_done = st[1];
    if (err_bits) *err_bits = st[0];
    return st[0] ? set_error(DNN_HIP_EDEVICE, "static decode: error bits %#x (1: a wait timed out, 2: no room for the steps)", st[0])
                 : DNN_HIP_OK;
}

}  // extern "C"
