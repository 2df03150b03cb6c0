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
    "c3": (8192, 768, 12, 12, 2048, 32, 32),
    "c2b8": (8192, 768, 12, 12, 2048, 32, 8),
}
SEED = {"c1": 1, "c2": 2, "c3": 3, "c2b8": 2}
KERNELS = {3: "decode_v3<NB,DC>", 4: "decode_v4<NB,DC>", 5: "decode_v5<NB,DC>",
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

    def __init__(self, ptr, V):
        self.ptr = C.c_void_p(ptr)
        self.V = V


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
    return ctx, lm, DeviceModel(dm, V)


def prompts(L, cfg, V, P, B):
    import numpy as np
    r = L.dnn_rng_seed(SEED[cfg] + 100)
    ids = [[L.dnn_rng_uniform_int(C.byref(r), V) for _ in range(P)] for _ in range(B)]
    return np.array(ids, dtype=np.int32).T.copy()     # [P][B]


def weight_floats(V, D, Ly, F):
    per_layer = D * 3 * D + 3 * D + D * D + D + 2 * D + 2 * (D * F + F) + F * D + D
    return V * D + Ly * per_layer + D + V


def step_bytes(V, D, Ly, F, positions, B):
    """Algorithmic HBM bytes of the decode steps whose new tokens sit at
    `positions` (0-based, S = pos+1 cached keys attended): every weight once per
    step, each row's K and V history read once per layer, one K and V row written."""
    w = 4 * weight_floats(V, D, Ly, F)
    total = 0
    for p in positions:
        kv_read = Ly * 2 * (p + 1) * D * 4 * B
        kv_write = Ly * 2 * D * 4 * B
        total += w + kv_read + kv_write
    return total


def measured_traffic(cfg, positions):
    """HBM bytes of this launch from the committed rocprofv3 --pmc summary of
    the same workload (profiles/traffic_<cfg>.json: FETCH_SIZE + WRITE_SIZE
    per step, scaled by a copy kernel of known size), or None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic_%s.json" % cfg)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return int(round(t["hbm_bytes_per_step"] * len(positions)))


def cpu_baseline(cfg, budget_tokens):
    """The reference itself (oracle/_ref/ref_bench, built from its sources), one
    thread, on a bounded sample of the same model: 4-token prompt, then
    `budget_tokens` greedy steps; falls back to the oracle port if absent."""
    V, D, Ly, H, F, _, _ = CONFIGS[cfg]
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_bench")
    env = dict(os.environ, OMP_NUM_THREADS="1")
    sample = "%s weights, 4-token prompt then %d greedy tokens, batch 1" % (cfg.upper(), budget_tokens)
    if os.path.exists(exe):
        out = subprocess.check_output([exe, str(V), str(D), str(Ly), str(H), str(F), "1088",
                                       str(SEED[cfg]), "4", str(budget_tokens)], env=env, text=True, timeout=600)
        r = json.loads(out.strip().splitlines()[-1])
        return {"value": round(r["tok_per_s"], 3), "unit": "tokens/s", "cores": 1, "kind": "reference",
                "sample": sample + " (masc-it/dnn.c built from its sources, NO_CBLAS scalar path)"}
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    m = O.Model(V, D, Ly, H, F, 1088, seed=SEED[cfg])
    p = O.prompt_ids(SEED[cfg] + 100, V, 4)
    t0 = time.perf_counter()
    m.generate(p, 1)
    t_p = time.perf_counter() - t0
    t0 = time.perf_counter()
    m.generate(p, budget_tokens)
    t_all = time.perf_counter() - t0
    return {"value": round((budget_tokens - 1) / (t_all - t_p), 3), "unit": "tokens/s", "cores": 1,
            "kind": "port", "sample": sample + " (oracle/dnn_oracle.c restatement)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--grid", type=int, default=0, help="persistent-kernel workgroups (0 = one per CU)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="after the timed decode, copy a MIB-sized device buffer 3 times (a plain copy kernel of "
                         "known size, the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--cpu-tokens", type=int, default=24)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (one-GPU boxes); --gpus %d is not supported" % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    V, D, Ly, H, F, P, B = CONFIGS[args.config]
    max_seq = P + args.warmup + args.steps + 1
    L = host_lib()
    dnn_amd.check(dnn_amd.hip().dnn_hip_init(0))
    ctx, lm, dm = build_model(L, args.config, max(max_seq, 1088))
    s = dnn_amd.HipSession(dm, B, max_seq)
    if args.grid:
        s.set_grid(args.grid)
    feed = prompts(L, args.config, V, P, B)
    ids, _ = s.decode(feed, P)                      # prompt, one token per step
    if args.warmup:
        ids, _ = s.decode(ids[-1:], args.warmup)    # warmup (greedy)
    start_pos = int(s.lengths()[0])
    t0 = time.perf_counter()
    ids, _ = s.decode(ids[-1:], args.steps)         # timed: exactly --steps greedy steps
    wall = time.perf_counter() - t0
    dev_ms = s.last_ms()
    assert ids.shape[0] == args.steps
    positions = range(start_pos, start_pos + args.steps)
    nbytes = step_bytes(V, D, Ly, F, positions, B)
    achieved = nbytes / (dev_ms * 1e-3) / 1e9
    tok_s = B * args.steps / wall
    line = {
        "metric": "decode tokens/sec @1 MI355X (B=1 and B=32) + % of HBM-bandwidth roofline",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,0.02) weights, uniform-random prompt",
        "config": {"workload": "%s greedy decode, batch %d" % (args.config.upper(), B),
                   "vocab": V, "d_model": D, "layers": Ly, "heads": H, "ffn": F, "prompt": P,
                   "batch": B, "positions": [start_pos, start_pos + args.steps - 1], "grid": s.grid()},
        "device_ms_per_step": round(dev_ms / args.steps, 5),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(achieved / 8000.0, 4), "traffic": None,
                     "kernel": "dnnhip::%s (one persistent launch = %d steps)" % (KERNELS.get(s.kernel(), "?"), args.steps),
                     "algorithmic_bytes_per_launch": nbytes},
    }
    traffic = measured_traffic(args.config, positions)
    if traffic is not None:
        line["roofline"]["traffic"] = traffic
    if args.copy_probe:
        import torch
        x = torch.empty(args.copy_probe << 18, dtype=torch.float32, device="cuda").fill_(1.0)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.config, args.cpu_tokens)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
