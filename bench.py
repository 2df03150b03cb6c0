#!/usr/bin/env python3
"""Decode throughput of the GPT token loop on one MI355X.

Workload ("C2"): decoder LM with V=8192, D=768,
12 layers, 12 heads (d_head 64), SwiGLU hidden 2048, tied lm_head, fp32,
N(0,0.02) random init, RoPE base 10000, a 32-token uniform-random prompt, then
greedy decode at batch 1.  A "step" is one decode token of every batch row.

The model is built through the product's own C API (libdnn_amd.so:
dnn_seed -> decoder_lm_create -> decoder_lm_init_normal -> decoder_lm_enable_rope)
and decoded through the C-ABI device layer (libdnn_hip.so).  The timed region is
exactly --steps greedy steps in one dnn_hip_decode call (one persistent-kernel
launch), weights and KV cache resident in HBM, prompt and warmup steps before it.

Prints one JSON line (rank 0, N=1 only).
"""
import argparse
import ctypes as C
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dnn.c_amd"))
import dnn_amd  # noqa: E402

CONFIGS = {
    # name: V, D, L, H, F, prompt, batch
    "c1": (128, 256, 4, 4, 683, 16, 1),
    "c2": (8192, 768, 12, 12, 2048, 32, 1),
    "c3": (8192, 768, 12, 12, 2048, 64, 32),
    "c2b2": (8192, 768, 12, 12, 2048, 32, 2),
    "c2b4": (8192, 768, 12, 12, 2048, 32, 4),
    "c2b8": (8192, 768, 12, 12, 2048, 32, 8),
}
SEED = {"c1": 1, "c2": 2, "c3": 3, "c2b2": 2, "c2b4": 2, "c2b8": 2, "c4": 4, "c5": 5}
KERNELS = {3: "decode_v3<NB,DC>",
           6: "batched engine: gemm_kernel / attn_kernel chain, one HIP graph replay per step"}


class Ctx(C.Structure):
    _fields_ = [("params", C.c_void_p), ("scratch", C.c_void_p), ("data", C.c_void_p)]


class Rng(C.Structure):
    _fields_ = [("s", C.c_uint64 * 2)]


def host_lib():
    L = C.CDLL(dnn_amd.AMD_LIB)
    L.dnn_ctx_init.argtypes = [C.POINTER(Ctx), C.c_size_t, C.c_size_t, C.c_size_t]
    L.dnn_seed.argtypes = [C.c_uint64]
    L.decoder_lm_create.argtypes = [C.c_void_p] + [C.c_int] * 6
    L.decoder_lm_create.restype = C.c_void_p
    L.decoder_lm_init_normal.argtypes = [C.c_void_p, C.c_float]
    L.decoder_lm_enable_rope.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_float]
    L.decoder_lm_device_model.argtypes = [C.c_void_p]
    L.decoder_lm_device_model.restype = C.c_void_p
    L.dnn_rng_seed.argtypes = [C.c_uint64]
    L.dnn_rng_seed.restype = Rng
    L.dnn_rng_uniform_int.argtypes = [C.POINTER(Rng), C.c_int]
    return L


class DeviceModel:
    """The host library's HBM mirror, shaped like dnn_amd.HipModel for sessions."""

    def __init__(self, ptr, V, D=0):
        self.ptr = C.c_void_p(ptr)
        self.V = V
        self.D = D


def build_model(L, cfg, max_seq):
    V, D, Ly, H, F, P, B = CONFIGS[cfg]
    ctx = Ctx()
    n_params = V * D + Ly * (4 * D * D + 3 * D * F + 8 * D + 2 * F) + 2 * V + D
    assert L.dnn_ctx_init(C.byref(ctx), n_params * 4 + (256 << 20), 16 << 20, 64 << 20) == 0
    L.dnn_seed(SEED[cfg])
    lm = L.decoder_lm_create(ctx.params, V, D, Ly, H, D // H, F)
    L.decoder_lm_init_normal(lm, 0.02)
    L.decoder_lm_enable_rope(ctx.params, lm, max_seq, 10000.0)
    dm = L.decoder_lm_device_model(lm)
    return ctx, lm, DeviceModel(dm, V, D)


def prompts(L, cfg, V, P, B):
    import numpy as np
    r = L.dnn_rng_seed(SEED[cfg] + 100)
    ids = [[L.dnn_rng_uniform_int(C.byref(r), V) for _ in range(P)] for _ in range(B)]
    return np.array(ids, dtype=np.int32).T.copy()     # [P][B]


def weight_floats(V, D, Ly, F):
    per_layer = D * 3 * D + 3 * D + D * D + D + 2 * D + 2 * (D * F + F) + F * D + D
    return V * D + Ly * per_layer + D + V


def step_bytes(V, D, Ly, F, positions, B, bf16=False):
    """Algorithmic HBM bytes of the decode steps whose new tokens sit at
    `positions` (0-based, S = pos+1 cached keys attended): every weight once per
    step (the matrices at 2 bytes each for bf16 weights), each row's K and V
    history read once per layer, one K and V row written.  `positions` holds one
    position per step for B rows at the same position, or (per-row lengths) one
    list of B positions per step."""
    w = 4 * weight_floats(V, D, Ly, F)
    if bf16:
        mats = V * D + Ly * (3 * D * D + D * D + 3 * D * F)
        w -= 2 * mats
    total = 0
    for p in positions:
        rows = list(p) if hasattr(p, "__len__") else [p] * B
        total += w
        for q in rows:
            total += Ly * 2 * (q + 1) * D * 4 + Ly * 2 * D * 4
    return total


def measured_traffic(cfg, positions):
    """HBM bytes of this launch from the committed rocprofv3 --pmc summary of
    the same workload (profiles/traffic_<cfg>.json: FETCH_SIZE + WRITE_SIZE of
    one launch, scaled by a copy kernel of known size).  Returns (bytes of this
    launch or None, the profiled launch's record): the bytes only when this
    launch covers exactly the profiled positions -- a launch over other
    positions moves other K/V bytes, and no figure is extrapolated."""
    path = os.path.join(ROOT, "profiles", "traffic_%s.json" % cfg)
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    rec = {k: t[k] for k in ("positions", "steps", "hbm_bytes", "algorithmic_bytes", "profile") if k in t}
    if list(t.get("positions", [])) == [positions[0], positions[-1]]:
        return int(t["hbm_bytes"]), rec
    return None, rec


def host_identity():
    """The CPU the baseline ran on: nproc, the lscpu model name, OMP_NUM_THREADS."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model, "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def ref_bench(cfg, prompt, new_tokens, seed=None):
    """One run of oracle/_ref/ref_bench (the reference built from its own
    sources, greedy decoder_lm_generate with the KV cache, one thread):
    returns its JSON record, or None where the reference build is absent."""
    V, D, Ly, H, F = CONFIGS[cfg][:5]
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_bench")
    if not os.path.exists(exe):
        return None
    env = dict(os.environ, OMP_NUM_THREADS="1")
    out = subprocess.check_output([exe, str(V), str(D), str(Ly), str(H), str(F), "1088",
                                   str(SEED[cfg] if seed is None else seed), str(prompt), str(new_tokens)],
                                  env=env, text=True, timeout=600)
    return json.loads(out.strip().splitlines()[-1])


def cpu_baseline(cfg, budget_tokens, prompt=32):
    """The reference itself (oracle/_ref/ref_bench), one thread, on a bounded
    sample of the same workload: the same model and seed, a `prompt`-token
    prompt, then `budget_tokens` greedy steps (the generation rate excludes the
    prompt); falls back to the oracle port if the reference build is absent."""
    V, D, Ly, H, F, _, _ = CONFIGS[cfg]
    sample = "%s weights, %d-token prompt then %d greedy tokens (positions %d..%d), batch 1" % (
        cfg.upper(), prompt, budget_tokens, prompt, prompt + budget_tokens - 1)
    r = ref_bench(cfg, prompt, budget_tokens)
    if r is not None:
        return {"value": round(r["tok_per_s"], 3), "unit": "tokens/s", "cores": 1, "kind": "reference",
                "sample": sample + " (masc-it/dnn.c built from its sources, NO_CBLAS scalar path)",
                "host": host_identity()}
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    m = O.Model(V, D, Ly, H, F, 1088, seed=SEED[cfg])
    p = O.prompt_ids(SEED[cfg] + 100, V, prompt)
    t0 = time.perf_counter()
    m.generate(p, 1)
    t_p = time.perf_counter() - t0
    t0 = time.perf_counter()
    m.generate(p, budget_tokens)
    t_all = time.perf_counter() - t0
    return {"value": round((budget_tokens - 1) / (t_all - t_p), 3), "unit": "tokens/s", "cores": 1,
            "kind": "port", "sample": sample + " (oracle/dnn_oracle.c restatement)", "host": host_identity()}


def cpu_baseline_batched(cfg, B, prompt, new_tokens):
    """The reference cannot batch generation (gpt.c:264): B independent
    batch-1 generations, timed serially (one process) and concurrently
    (min(B, 16) processes, one dnn_ctx each, one thread each).  Bounded
    sample: `prompt`-token prompts, `new_tokens` greedy tokens per sequence."""
    from concurrent.futures import ThreadPoolExecutor
    serial = ref_bench(cfg, prompt, new_tokens)
    if serial is None:
        return None
    n_par = max(1, min(B, 16, os.cpu_count() or 1))
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=n_par) as ex:
        runs = list(ex.map(lambda i: ref_bench(cfg, prompt, new_tokens, seed=SEED[cfg] + 1000 + i), range(n_par)))
    wall = time.perf_counter() - t0
    agg = sum(r["tok_per_s"] for r in runs)
    return {"value": round(agg, 3), "unit": "tokens/s", "cores": n_par, "kind": "reference",
            "serial_value": round(serial["tok_per_s"], 3), "serial_cores": 1,
            "sample": "%d concurrent batch-1 generations (one process and thread each) of %s weights, "
                      "%d-token prompt then %d greedy tokens each; value = the sum of their generation rates "
                      "(wall %.1f s); serial_value = one such generation alone" % (
                          n_par, cfg.upper(), prompt, new_tokens, wall),
            "host": host_identity()}


def decode_run(L, cfg, steps, warmup, grid=0, bf16=False):
    """Greedy decode of CONFIGS[cfg]: prompt, warmup, then exactly `steps` timed
    steps in one dnn_hip_decode call (bf16: the same model with its weight
    matrices stored as bf16, W16A32).  Returns the measurement dict."""
    V, D, Ly, H, F, P, B = CONFIGS[cfg]
    max_seq = P + warmup + steps + 1
    ctx, lm, dm = build_model(L, cfg, max(max_seq, 1088))
    if bf16:
        L.decoder_lm_device_model_ex.argtypes = [C.c_void_p, C.c_int]
        L.decoder_lm_device_model_ex.restype = C.c_void_p
        dm = DeviceModel(L.decoder_lm_device_model_ex(lm, dnn_amd.WEIGHTS_BF16), V, D)
    s = dnn_amd.HipSession(dm, B, max_seq)
    if grid:
        s.set_grid(grid)
    feed = prompts(L, cfg, V, P, B)
    ids, _ = s.decode(feed, P)                      # prompt, one token per step
    first_ids = ids[-1].copy()
    if warmup:
        ids, _ = s.decode(ids[-1:], warmup)         # warmup (greedy)
    start_pos = int(s.lengths()[0])
    t0 = time.perf_counter()
    ids, _ = s.decode(ids[-1:], steps)              # timed: exactly `steps` greedy steps
    wall = time.perf_counter() - t0
    dev_ms = s.last_ms()
    assert ids.shape[0] == steps
    positions = range(start_pos, start_pos + steps)
    nbytes = step_bytes(V, D, Ly, F, positions, B, bf16)
    achieved = nbytes / (dev_ms * 1e-3) / 1e9
    kern = s.kernel()
    # time to the first generated token: the prompt again on the reset
    # session, one token per step as decoder_lm_generate feeds it
    # (gpt.c:306-344); its last step emits the first greedy token
    s.reset()
    t0 = time.perf_counter()
    again, _ = s.decode(feed, P)
    ttft = time.perf_counter() - t0
    ttft_dev = s.last_ms()
    assert (again[-1] == first_ids).all()
    # the same prompt through the batched prefill (all prompt rows at once on
    # the MFMA engine; the same cache, then decode continues from it): its
    # first token, and whether it is the token-by-token one (it may differ
    # only at a near-tie: the summation order differs)
    s.reset()
    s.prefill(ids=feed.T.copy())                    # warm-up (the engine's buffers and weight copy)
    s.reset()
    t0 = time.perf_counter()
    nxt, _ = s.prefill(ids=feed.T.copy())
    pre_wall = time.perf_counter() - t0
    first = {"prompt_tokens": P, "ms": round(ttft * 1e3, 3), "device_ms": round(ttft_dev, 3),
             "batched_prefill": {"ms": round(pre_wall * 1e3, 3), "device_ms": round(s.last_ms(), 3),
                                 "same_token": bool((nxt == first_ids).all())}}
    return {
        "first_token": first,
        "tok_s": B * steps / wall, "ms_per_step": wall * 1e3 / steps, "device_ms_per_step": dev_ms / steps,
        "achieved": achieved, "nbytes": nbytes, "kernel": kern, "grid": s.grid(), "B": B,
        "positions": [start_pos, start_pos + steps - 1], "P": P,
        "kernel_desc": ("dnnhip::%s (one persistent launch = %d steps)" % (KERNELS[kern], steps)) if kern in (3, 4, 5)
        else "dnnhip::%s (%d replays)" % (KERNELS.get(kern, "?"), steps),
    }


def run_c3(L, steps=256):
    """the C2 model at batch 32; every row has its own
    uniform-random 64-token prompt cut to a length drawn uniformly from
    [16, 64] (per-row lengths), prefilled at once, then `steps` greedy steps of
    all rows timed.  The whole workload runs twice on one session (the first
    pass warms buffers and captures the step graph; reset in between): the
    second pass is timed and must emit the first pass's tokens."""
    import numpy as np
    V, D, Ly, H, F, P, B = CONFIGS["c3"]
    ctx, lm, dm = build_model(L, "c3", P + steps + 1)
    r = L.dnn_rng_seed(SEED["c3"] + 100)
    ids = np.array([[L.dnn_rng_uniform_int(C.byref(r), V) for _ in range(P)] for _ in range(B)], dtype=np.int32)
    lens = np.array([16 + L.dnn_rng_uniform_int(C.byref(r), P - 16 + 1) for _ in range(B)], dtype=np.int32)
    s = dnn_amd.HipSession(dm, B, P + steps + 1)
    runs = []
    for rep in range(2):
        s.reset()
        t0 = time.perf_counter()
        nxt, _ = s.prefill(ids=ids, n_ids=lens)
        pre_wall = time.perf_counter() - t0
        pre_ms = s.last_ms()
        t0 = time.perf_counter()
        out, _ = s.decode(nxt, steps)
        wall = time.perf_counter() - t0
        runs.append((out, wall, s.last_ms(), pre_wall, pre_ms))
    assert np.array_equal(runs[0][0], runs[1][0]), "c3: the timed pass emitted other tokens than the first"
    out, wall, dev_ms, pre_wall, pre_ms = runs[1]
    positions = [[int(lens[b]) + t for b in range(B)] for t in range(steps)]
    nbytes = step_bytes(V, D, Ly, F, positions, B)
    return {
        "tok_s": B * steps / wall, "ms_per_step": wall * 1e3 / steps, "device_ms_per_step": dev_ms / steps,
        "achieved": nbytes / (dev_ms * 1e-3) / 1e9, "nbytes": nbytes, "kernel": s.kernel(), "grid": 0, "B": B,
        "P": P, "prompt_lens": [int(lens.min()), int(lens.max())],
        "positions": [int(lens.min()), int(lens.max()) + steps - 1],
        "kernel_desc": "dnnhip::%s (%d replays)" % (KERNELS.get(s.kernel(), "?"), steps),
        "prefill": {"tokens": int(lens.sum()), "ms": round(pre_ms, 3), "wall_ms": round(pre_wall * 1e3, 3)},
        "workload": "C3: batch 32, 64-token uniform-random prompts cut to lengths U[16,64] (%d..%d), "
                    "ragged prefill, then %d greedy steps of every row" % (lens.min(), lens.max(), steps),
    }


def copy_probe(nbytes):
    """Three device-to-device copies of nbytes (the runtime's blit kernel): a
    plain copy of known size, the scale for the FETCH_SIZE / WRITE_SIZE counters."""
    rt = C.CDLL("libamdhip64.so")
    rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    rt.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rt.hipFree.argtypes = [C.c_void_p]
    a, b = C.c_void_p(), C.c_void_p()
    assert rt.hipMalloc(C.byref(a), nbytes) == 0 and rt.hipMalloc(C.byref(b), nbytes) == 0
    assert rt.hipMemset(a, 1, nbytes) == 0
    for _ in range(3):
        assert rt.hipMemcpy(b, a, nbytes, 3) == 0          # hipMemcpyDeviceToDevice
    assert rt.hipDeviceSynchronize() == 0
    rt.hipFree(a)
    rt.hipFree(b)


def prefill_flops(D, Ly, F, V, lens_new, lens_old=None):
    """fp32 FLOPs of a multi-token prefill: the GEMMs of every new row (qkv,
    out, gate/up, down) plus causal attention (QK^T and PV over the visible
    keys), plus the lm_head of each sequence's last row."""
    per_row = 2 * Ly * (3 * D * D + D * D + 2 * D * F + F * D)
    total = 0
    for i, n in enumerate(lens_new):
        old = lens_old[i] if lens_old else 0
        vis = sum(old + t + 1 for t in range(n))
        total += n * per_row + Ly * 4 * D * vis + 2 * D * V
    return total


def run_c4(L, args):
    """8 sequences of 1024 uniform-random tokens prefilled
    at once (MFMA GEMMs, tiled causal attention writing the KV cache), then 64
    greedy decode steps of all 8 rows."""
    V, D, Ly, H, F = 8192, 768, 12, 12, 2048
    B, T, steps = 8, 1024, args.steps if args.steps != 512 else 64
    CONFIGS["c4"] = (V, D, Ly, H, F, T, B)
    ctx, lm, dm = build_model(L, "c4", T + steps + 1)
    import numpy as np
    r = L.dnn_rng_seed(SEED["c4"] + 100)
    ids = np.array([[L.dnn_rng_uniform_int(C.byref(r), V) for _ in range(T)] for _ in range(B)], dtype=np.int32)
    s = dnn_amd.HipSession(dm, B, T + steps + 1)
    s.prefill(ids=ids)                              # warm-up pass (buffers, code)
    s.reset()
    t0 = time.perf_counter()
    nxt, _ = s.prefill(ids=ids)
    pre_wall = time.perf_counter() - t0
    pre_ms = s.last_ms()
    t0 = time.perf_counter()
    out, _ = s.decode(nxt, steps)
    wall = time.perf_counter() - t0
    dev_ms = s.last_ms()
    positions = range(T, T + steps)
    nbytes = step_bytes(V, D, Ly, F, positions, B)
    fl = prefill_flops(D, Ly, F, V, [T] * B)
    return {
        "tok_s": B * steps / wall, "ms_per_step": wall * 1e3 / steps, "device_ms_per_step": dev_ms / steps,
        "achieved": nbytes / (dev_ms * 1e-3) / 1e9, "nbytes": nbytes, "kernel": s.kernel(), "B": B, "P": T,
        "positions": [T, T + steps - 1], "grid": 0,
        "kernel_desc": ("dnnhip::%s (one persistent launch = %d steps)" if s.kernel() in (3, 4, 5)
                        else "dnnhip::%s (%d replays)") % (KERNELS.get(s.kernel(), "?"), steps),
        "prefill": {"tokens": B * T, "ms": round(pre_ms, 3), "wall_ms": round(pre_wall * 1e3, 3),
                    "tokens_per_s": round(B * T / (pre_ms * 1e-3), 1), "flops": fl,
                    "tflops": round(fl / (pre_ms * 1e-3) / 1e12, 2), "mfma_fp32_peak_tflops": 157.3,
                    "frac": round(fl / (pre_ms * 1e-3) / 1e12 / 157.3, 4)},
    }


def run_c5(L, args):
    """prefix-LM (VLM-shaped) decode, bf16 weights: 64 rows,
    196 bidirectional patch-embedding rows ~N(0,1) (d=512) then 1..4 causal text
    tokens (sequence lengths 197..200) prefilled at once, then 16 greedy steps."""
    import numpy as np
    V, D, Ly, H, F = 1024, 512, 8, 8, 1024
    B, I, steps = 64, 196, args.steps if args.steps != 512 else 16
    CONFIGS["c5"] = (V, D, Ly, H, F, I + 4, B)
    max_seq = I + 4 + steps + 1
    ctx = Ctx()
    n_params = V * D + Ly * (4 * D * D + 3 * D * F + 8 * D + 2 * F) + 2 * V + D
    assert L.dnn_ctx_init(C.byref(ctx), n_params * 4 + (64 << 20), 16 << 20, 64 << 20) == 0
    L.dnn_seed(SEED["c5"])
    lm = L.decoder_lm_create(ctx.params, V, D, Ly, H, D // H, F)
    L.decoder_lm_init_normal(lm, 0.02)
    L.decoder_lm_enable_rope(ctx.params, lm, max_seq, 10000.0)
    L.decoder_lm_device_model_ex.argtypes = [C.c_void_p, C.c_int]
    L.decoder_lm_device_model_ex.restype = C.c_void_p
    dm = DeviceModel(L.decoder_lm_device_model_ex(lm, dnn_amd.WEIGHTS_BF16), V, D)
    r = L.dnn_rng_seed(SEED["c5"] + 100)
    L.dnn_rng_normal.argtypes = [C.POINTER(Rng)]
    L.dnn_rng_normal.restype = C.c_float
    emb = np.array([L.dnn_rng_normal(C.byref(r)) for _ in range(B * I * D)], dtype=np.float32).reshape(B, I, D)
    n_ids = np.array([1 + L.dnn_rng_uniform_int(C.byref(r), 4) for _ in range(B)], dtype=np.int32)
    ids = np.array([[L.dnn_rng_uniform_int(C.byref(r), V) for _ in range(4)] for _ in range(B)], dtype=np.int32)
    s = dnn_amd.HipSession(dm, B, max_seq)
    s.prefill(ids=ids, n_ids=n_ids, embeds=emb, mode=1, prefix_len=I)     # warm-up pass
    s.reset()
    t0 = time.perf_counter()
    nxt, _ = s.prefill(ids=ids, n_ids=n_ids, embeds=emb, mode=1, prefix_len=I)
    pre_wall = time.perf_counter() - t0
    pre_ms = s.last_ms()
    lens = [int(x) for x in s.lengths()]
    t0 = time.perf_counter()
    out, _ = s.decode(nxt, steps)
    wall = time.perf_counter() - t0
    dev_ms = s.last_ms()
    # algorithmic bytes per step: bf16 weight matrices, fp32 biases / gammas,
    # each row's fp32 K/V history (its own length) read, one K/V row written
    mats = V * D + Ly * (3 * D * D + D * D + 2 * D * F + F * D)
    vecs = Ly * (3 * D + D + 2 * D + 2 * F + D) + D + V
    nbytes = 0
    for t in range(steps):
        nbytes += 2 * mats + 4 * vecs + sum(Ly * 2 * (ln + t + 1) * D * 4 + Ly * 2 * D * 4 for ln in lens)
    fl = prefill_flops(D, Ly, F, V, [I + int(n) for n in n_ids])
    return {
        "tok_s": B * steps / wall, "ms_per_step": wall * 1e3 / steps, "device_ms_per_step": dev_ms / steps,
        "achieved": nbytes / (dev_ms * 1e-3) / 1e9, "nbytes": nbytes, "kernel": s.kernel(), "B": B, "P": I,
        "positions": [min(lens), max(lens) + steps - 1], "grid": 0, "dtype": "bf16 weights, f32 arithmetic (W16A32)",
        "kernel_desc": "dnnhip::%s (%d replays)" % (KERNELS.get(s.kernel(), "?"), steps),
        "prefill": {"tokens": int(sum(lens)), "ms": round(pre_ms, 3), "wall_ms": round(pre_wall * 1e3, 3),
                    "tokens_per_s": round(sum(lens) / (pre_ms * 1e-3), 1), "flops": fl,
                    "tflops": round(fl / (pre_ms * 1e-3) / 1e12, 2), "mfma_fp32_peak_tflops": 157.3,
                    "frac": round(fl / (pre_ms * 1e-3) / 1e12 / 157.3, 4)},
    }


def summary(r):
    out = {"tokens_per_s": round(r["tok_s"], 2), "ms_per_step": round(r["ms_per_step"], 5),
           "batch": r["B"], "roofline_achieved_GBps": round(r["achieved"], 1),
           "roofline_frac": round(r["achieved"] / 8000.0, 4), "kernel": r["kernel_desc"]}
    for k in ("prefill", "first_token"):
        if k in r:
            out[k] = r[k]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS) + ["c4", "c5"])
    ap.add_argument("--c3-steps", type=int, default=256, help="greedy steps of the C3 (batch 32) line")
    ap.add_argument("--grid", type=int, default=0, help="persistent-kernel workgroups (0 = one per CU)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="after the timed decode, copy a MIB-sized device buffer 3 times (a plain copy kernel of "
                         "known size, the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--cpu-tokens", type=int, default=24)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="the headline workload only (no C3 / bf16 lines)")
    ap.add_argument("--bf16", action="store_true", help="the decode workload with bf16 weight matrices (W16A32)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (one-GPU boxes); --gpus %d is not supported" % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    L = host_lib()
    dnn_amd.check(dnn_amd.hip().dnn_hip_init(0))
    cfg = args.config
    if cfg == "c3":
        r = run_c3(L, args.c3_steps if args.steps == 512 else args.steps)
    elif cfg == "c4":
        r = run_c4(L, args)
    elif cfg == "c5":
        r = run_c5(L, args)
    else:
        r = decode_run(L, cfg, args.steps, args.warmup, args.grid, bf16=args.bf16)
    V, D, Ly, H, F, P, B = CONFIGS[cfg]
    steps = len(range(r["positions"][0], r["positions"][1] + 1)) if cfg not in ("c5",) else (
        args.steps if args.steps != 512 else 16)
    line = {
        "metric": "decode tokens/sec @1 MI355X (B=1 and B=32) + % of HBM-bandwidth roofline",
        "value": round(r["tok_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights / f32" if cfg == "c5" or args.bf16 else "f32",
        "data": "synthetic: seeded N(0,0.02) weights, uniform-random prompt" + (
            ", N(0,1) patch embeddings" if cfg == "c5" else ""),
        "config": {"workload": r.get("workload", "%s greedy decode, batch %d" % (cfg.upper(), r["B"])),
                   "vocab": V, "d_model": D, "layers": Ly, "heads": H, "ffn": F, "prompt": r["P"],
                   "batch": r["B"], "positions": r["positions"], "grid": r["grid"]},
        "device_ms_per_step": round(r["device_ms_per_step"], 5),
        "roofline": {"bound": "hbm", "achieved": round(r["achieved"], 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(r["achieved"] / 8000.0, 4), "traffic": None,
                     "kernel": r["kernel_desc"], "algorithmic_bytes_per_launch": r["nbytes"]},
    }
    for k in ("prefill", "first_token"):
        if k in r:
            line[k] = r[k]
    positions = range(r["positions"][0], r["positions"][1] + 1)
    traffic, prof = measured_traffic(cfg, positions) if cfg not in ("c4", "c5") and not args.bf16 else (None, None)
    line["roofline"]["traffic"] = traffic
    if prof is not None:
        line["roofline"]["traffic_profiled_launch"] = prof
    if cfg == "c2" and not args.no_extra:
        # the metric's second batch size, on the batched engine
        r3 = run_c3(L, args.c3_steps)
        line["c3_batch32"] = summary(r3)
        line["c3_batch32"]["workload"] = r3["workload"]
        if not args.no_cpu_baseline:
            line["c3_batch32"]["cpu_baseline"] = cpu_baseline_batched("c3", 32, 16, 8)
        # the bf16-weight variant of the headline (north_star: reported
        # separately, with its tolerance)
        rb = decode_run(L, cfg, args.steps, args.warmup, args.grid, bf16=True)
        line["c2_bf16"] = summary(rb)
        line["c2_bf16"]["workload"] = "C2 greedy decode, batch 1, weight matrices stored as bf16 (W16A32)"
        line["c2_bf16"]["dtype"] = "bf16 weights / f32"
        line["c2_bf16"]["tolerance"] = ("against fp32 arithmetic on the bf16-rounded weights: logits max-abs 1e-3 "
                                        "and relative 1e-4, greedy tokens identical "
                                        "(tests/test_configs_gpu.py::test_c2_bf16_weights_every_step_logits)")
    if args.copy_probe:
        copy_probe(args.copy_probe << 20)
    if not args.no_cpu_baseline and cfg in CONFIGS and cfg not in ("c3", "c4", "c5"):
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens, prompt=min(P, 32))
    elif not args.no_cpu_baseline and cfg == "c3":
        line["cpu_baseline"] = cpu_baseline_batched("c3", 32, 16, 8)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
