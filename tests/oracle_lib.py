"""ctypes binding of oracle/_build/liboracle.so -- the CPU checker.

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it to check or time against; the product never does.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "_build", "liboracle.so")

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int)


class Cfg(C.Structure):
    _fields_ = [("V", C.c_int), ("D", C.c_int), ("L", C.c_int), ("H", C.c_int),
                ("dk", C.c_int), ("F", C.c_int), ("max_seq", C.c_int),
                ("rope_base", C.c_float)]


class Rng(C.Structure):
    _fields_ = [("s", C.c_uint64 * 2)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
        L = C.CDLL(LIB_PATH)
        L.orc_rng_seed.argtypes = [C.POINTER(Rng), C.c_uint64]
        L.orc_rng_uniform.argtypes = [C.POINTER(Rng)]
        L.orc_rng_uniform.restype = C.c_float
        L.orc_rng_normal.argtypes = [C.POINTER(Rng)]
        L.orc_rng_normal.restype = C.c_float
        L.orc_rng_uniform_int.argtypes = [C.POINTER(Rng), C.c_int]
        L.orc_model_create.argtypes = [C.POINTER(Cfg)]
        L.orc_model_create.restype = C.c_void_p
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_model_n_params.argtypes = [C.c_void_p]
        L.orc_model_param.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_longlong)]
        L.orc_model_param.restype = f32p
        L.orc_model_init_create.argtypes = [C.c_void_p, C.c_uint64]
        L.orc_model_init_synthetic.argtypes = [C.c_void_p, C.c_float]
        L.orc_model_init_gpt2.argtypes = [C.c_void_p]
        L.orc_model_rope.argtypes = [C.c_void_p, C.c_int, C.c_float]
        L.orc_generate.argtypes = [C.c_void_p, i32p, C.c_int, C.c_int, C.c_int, i32p, f32p]
        L.orc_forward_full.argtypes = [C.c_void_p, i32p, C.c_int, f32p]
        L.orc_state_create.argtypes = [C.c_void_p, C.c_int]
        L.orc_state_create.restype = C.c_void_p
        L.orc_state_free.argtypes = [C.c_void_p]
        L.orc_forward_cached.argtypes = [C.c_void_p, f32p, C.c_int, C.c_int, C.c_int]
        L.orc_state_kv.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, f32p]
        L.orc_head.argtypes = [C.c_void_p, f32p, C.c_int, f32p]
        L.orc_embed.argtypes = [C.c_void_p, i32p, C.c_int, f32p]
        L.orc_argmax.argtypes = [f32p, C.c_int]
        L.orc_matmul_add.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_rms_norm.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
        L.orc_rope_rows.argtypes = [f32p, C.c_int, C.c_int, f32p, f32p]
        L.orc_swiglu.argtypes = [f32p, f32p, f32p, C.c_int]
        L.orc_fnv.argtypes = [C.c_void_p, C.c_size_t]
        L.orc_fnv.restype = C.c_uint64
        L.orc_model_rope_cos.argtypes = [C.c_void_p]
        L.orc_model_rope_cos.restype = f32p
        L.orc_model_rope_sin.argtypes = [C.c_void_p]
        L.orc_model_rope_sin.restype = f32p
        L.orc_model_rope_rows.argtypes = [C.c_void_p]
        _lib = L
    return _lib


def fp(a):
    return a.ctypes.data_as(f32p)


def ip(a):
    return a.ctypes.data_as(i32p)


class Model:
    """Oracle model built the way the parity configs are built."""

    def __init__(self, V, D, L, H, F, max_seq, seed, init="synthetic", std=0.02, rope_base=10000.0):
        self.cfg = Cfg(V, D, L, H, D // H, F, max_seq, 0.0)
        self.V, self.D, self.L, self.H, self.F = V, D, L, H, F
        self.ptr = lib().orc_model_create(C.byref(self.cfg))
        lib().orc_model_init_create(self.ptr, seed)
        if init == "synthetic":
            lib().orc_model_init_synthetic(self.ptr, std)
        elif init == "gpt2":
            lib().orc_model_init_gpt2(self.ptr)
        elif init != "create":
            raise ValueError(init)
        if rope_base:
            lib().orc_model_rope(self.ptr, max_seq, rope_base)

    def params(self):
        out = []
        for i in range(lib().orc_model_n_params(self.ptr)):
            n = C.c_longlong()
            p = lib().orc_model_param(self.ptr, i, C.byref(n))
            out.append(np.ctypeslib.as_array(p, shape=(n.value,)).copy())
        return out

    def param_view(self, i):
        """Parameter i of the oracle model (0: embedding, then 12 per layer,
        then the final gamma and the lm_head bias) as a writable view."""
        n = C.c_longlong()
        p = lib().orc_model_param(self.ptr, i, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def round_weights_bf16(self):
        """Rounds every weight matrix (embedding, qkv, out, gate, up, down) to
        bf16 in place (round to nearest even, stored back as fp32): the W16A32
        model a bf16-weight device model computes.  Biases and gammas stay."""
        mats = [0] + [1 + 12 * l + k for l in range(self.L) for k in (0, 2, 6, 8, 10)]
        for i in mats:
            n = C.c_longlong()
            p = lib().orc_model_param(self.ptr, i, C.byref(n))
            a = np.ctypeslib.as_array(p, shape=(n.value,))
            u = a.view(np.uint32)
            r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
            u[:] = r

    def rope_tables(self):
        rows = lib().orc_model_rope_rows(self.ptr)
        if rows == 0:
            return None
        half = self.D // self.H // 2
        cos = np.ctypeslib.as_array(lib().orc_model_rope_cos(self.ptr), shape=(rows, half)).copy()
        sin = np.ctypeslib.as_array(lib().orc_model_rope_sin(self.ptr), shape=(rows, half)).copy()
        return cos, sin

    def generate(self, prompt, max_new, eos=258, want_logits=False):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(len(prompt) + max_new, dtype=np.int32)
        lg = np.zeros((max_new, self.V), dtype=np.float32) if want_logits else None
        n = lib().orc_generate(self.ptr, ip(prompt), len(prompt), max_new, eos, ip(out),
                               fp(lg) if want_logits else None)
        return (out[:n], lg[: n - len(prompt)]) if want_logits else out[:n]

    def forward_full(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        lg = np.zeros((len(ids), self.V), dtype=np.float32)
        lib().orc_forward_full(self.ptr, ip(ids), len(ids), fp(lg))
        return lg

    def __del__(self):
        try:
            lib().orc_model_free(self.ptr)
        except Exception:
            pass


class State:
    def __init__(self, model, max_seq):
        self.m = model
        self.ptr = lib().orc_state_create(model.ptr, max_seq)

    def forward(self, x, mode=0, prefix_len=0):
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        lib().orc_forward_cached(self.ptr, fp(x), x.shape[0], mode, prefix_len)
        return x

    def cache(self, layer, which, length):
        """[H][length][dk] rows of one layer's K (which 0) or V (which 1)."""
        out = np.zeros((self.m.H, length, self.m.D // self.m.H), dtype=np.float32)
        lib().orc_state_kv(self.ptr, layer, which, length, fp(out))
        return out

    def __del__(self):
        try:
            lib().orc_state_free(self.ptr)
        except Exception:
            pass


def embed(model, ids):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    x = np.zeros((len(ids), model.D), dtype=np.float32)
    lib().orc_embed(model.ptr, ip(ids), len(ids), fp(x))
    return x


def head(model, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    lg = np.zeros((x.shape[0], model.V), dtype=np.float32)
    lib().orc_head(model.ptr, fp(x), x.shape[0], fp(lg))
    return lg


def prompt_ids(seed, V, P):
    r = Rng()
    lib().orc_rng_seed(C.byref(r), seed)
    return np.array([lib().orc_rng_uniform_int(C.byref(r), V) for _ in range(P)], dtype=np.int32)


def fnv(a):
    a = np.ascontiguousarray(a)
    return "%016x" % lib().orc_fnv(a.ctypes.data, a.nbytes)
