"""Python binding of the C-ABI device layer (include/dnn_hip.h) via ctypes.

The product is the C/HIP libraries under dnn.c_amd/lib; this module only loads
them for the test suite and bench.py.  There is no fallback: if
lib/libdnn_hip.so is missing or fails to load, every call raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
HIP_LIB = os.path.join(LIB_DIR, "libdnn_hip.so")
AMD_LIB = os.path.join(LIB_DIR, "libdnn_amd.so")

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int)

# every symbol include/dnn_hip.h declares
HIP_SYMBOLS = [
    "dnn_hip_last_error", "dnn_hip_init", "dnn_hip_model_create", "dnn_hip_model_update",
    "dnn_hip_model_rope", "dnn_hip_model_destroy", "dnn_hip_session_create",
    "dnn_hip_session_reset", "dnn_hip_session_lengths", "dnn_hip_session_destroy",
    "dnn_hip_decode", "dnn_hip_generate", "dnn_hip_session_last_ms", "dnn_hip_session_set_grid",
    "dnn_hip_session_grid", "dnn_hip_session_kernel", "dnn_hip_session_att_splits", "dnn_hip_model_create_ex", "dnn_hip_prefill",
    "dnn_hip_block_forward", "dnn_hip_head_forward", "dnn_hip_embed", "dnn_hip_cache_read", "dnn_hip_rms_norm",
    "dnn_hip_linear", "dnn_hip_op_matmul_add", "dnn_hip_op_add", "dnn_hip_op_swiglu", "dnn_hip_op_rms_norm",
    "dnn_hip_op_rope", "dnn_hip_op_embedding", "dnn_hip_op_split_heads", "dnn_hip_op_merge_heads",
    "dnn_hip_op_linear", "dnn_hip_op_swiglu_ffn", "dnn_hip_op_cache_drop",
    "dnn_hip_kv_floats", "dnn_hip_decode_static", "dnn_hip_decode_static_status",
]

WEIGHTS_F32 = 0
WEIGHTS_BF16 = 1


class HipError(RuntimeError):
    pass


_hip = None


def hip():
    """Loads lib/libdnn_hip.so (raises if it is not built)."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB):
            raise HipError("%s is not built: run `make -C dnn.c_amd` (or __graft_entry__.build())" % HIP_LIB)
        L = C.CDLL(HIP_LIB)
        L.dnn_hip_last_error.restype = C.c_char_p
        L.dnn_hip_init.argtypes = [C.c_int]
        L.dnn_hip_model_create.argtypes = [C.c_int] * 6 + [C.POINTER(f32p), C.c_int, f32p, C.POINTER(C.c_void_p)]
        L.dnn_hip_model_update.argtypes = [C.c_void_p, C.POINTER(f32p), C.c_int]
        L.dnn_hip_model_rope.argtypes = [C.c_void_p, f32p, f32p, C.c_int]
        L.dnn_hip_model_destroy.argtypes = [C.c_void_p]
        L.dnn_hip_session_create.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        L.dnn_hip_session_reset.argtypes = [C.c_void_p]
        L.dnn_hip_session_lengths.argtypes = [C.c_void_p, i32p]
        L.dnn_hip_session_destroy.argtypes = [C.c_void_p]
        L.dnn_hip_decode.argtypes = [C.c_void_p, i32p, C.c_int, i32p, C.c_int, C.c_int, i32p, f32p, i32p]
        L.dnn_hip_generate.argtypes = [C.c_void_p, i32p, C.c_int, C.c_int, C.c_int, i32p, i32p]
        L.dnn_hip_session_last_ms.argtypes = [C.c_void_p, f32p]
        L.dnn_hip_session_set_grid.argtypes = [C.c_void_p, C.c_int]
        L.dnn_hip_session_grid.argtypes = [C.c_void_p, i32p]
        L.dnn_hip_session_kernel.argtypes = [C.c_void_p, i32p]
        L.dnn_hip_session_att_splits.argtypes = [C.c_void_p, i32p]
        L.dnn_hip_model_create_ex.argtypes = [C.c_int] * 6 + [C.POINTER(f32p), C.c_int, f32p, C.c_int,
                                                              C.POINTER(C.c_void_p)]
        L.dnn_hip_prefill.argtypes = [C.c_void_p, f32p, C.c_int, i32p, C.c_int, i32p, C.c_int, C.c_int, i32p, f32p]
        L.dnn_hip_block_forward.argtypes = [C.c_void_p, C.c_int, f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p]
        L.dnn_hip_head_forward.argtypes = [C.c_void_p, f32p, C.c_int, C.c_int, f32p]
        L.dnn_hip_embed.argtypes = [C.c_void_p, i32p, C.c_int, f32p]
        L.dnn_hip_cache_read.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, f32p]
        L.dnn_hip_rms_norm.argtypes = [C.c_void_p, f32p, f32p, C.c_int, C.c_int, C.c_float, f32p]
        _hip = L
    return _hip


def check(rc):
    if rc != 0:
        raise HipError("dnn_hip error %d: %s" % (rc, hip().dnn_hip_last_error().decode()))


def _fp(a):
    return a.ctypes.data_as(f32p)


def _ip(a):
    return a.ctypes.data_as(i32p)


class HipModel:
    """HBM mirror of a decoder LM given its parameters in module order."""

    def __init__(self, V, D, L, H, F, params, rope=None, dk=64, weights=WEIGHTS_F32):
        params = [np.ascontiguousarray(p, dtype=np.float32) for p in params]
        self._keep = params
        arr = (f32p * len(params))(*[_fp(p) for p in params])
        h = C.c_void_p()
        check(hip().dnn_hip_init(0))
        check(hip().dnn_hip_model_create_ex(V, D, L, H, dk, F, arr, len(params), None, weights, C.byref(h)))
        self.ptr = h
        self.V, self.D, self.L, self.H, self.F = V, D, L, H, F
        if rope is not None:
            cos, sin = [np.ascontiguousarray(t, dtype=np.float32) for t in rope]
            check(hip().dnn_hip_model_rope(self.ptr, _fp(cos), _fp(sin), cos.shape[0]))

    def generate(self, prompt, max_new, eos=258):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(len(prompt) + max_new, dtype=np.int32)
        n = C.c_int()
        check(hip().dnn_hip_generate(self.ptr, _ip(prompt), len(prompt), max_new, eos, _ip(out), C.byref(n)))
        return out[: n.value]

    def close(self):
        if getattr(self, "ptr", None):
            hip().dnn_hip_model_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipSession:
    def __init__(self, model, batch, max_seq):
        self.m = model
        self.B = batch
        h = C.c_void_p()
        check(hip().dnn_hip_session_create(model.ptr, batch, max_seq, C.byref(h)))
        self.ptr = h

    def grid(self):
        g = C.c_int()
        check(hip().dnn_hip_session_grid(self.ptr, C.byref(g)))
        return g.value

    def kernel(self):
        """3..6: the decode kernel of the last decode() call (6: the batched engine)."""
        k = C.c_int()
        check(hip().dnn_hip_session_kernel(self.ptr, C.byref(k)))
        return k.value

    def att_splits(self):
        """Workgroups per (row, head) of the last general-kernel launch's attention."""
        k = C.c_int()
        check(hip().dnn_hip_session_att_splits(self.ptr, C.byref(k)))
        return k.value

    def set_grid(self, n):
        check(hip().dnn_hip_session_set_grid(self.ptr, n))

    def decode(self, feed, n_steps, n_feed=None, eos=-1, want_logits=False):
        """feed: [n_feed_max][B] ints.  Returns (ids [steps][B], logits or None)."""
        feed = np.ascontiguousarray(feed, dtype=np.int32).reshape(-1, self.B)
        nf = None if n_feed is None else np.ascontiguousarray(n_feed, dtype=np.int32)
        ids = np.zeros((n_steps, self.B), dtype=np.int32)
        lg = np.zeros((n_steps, self.B, self.m.V), dtype=np.float32) if want_logits else None
        done = C.c_int()
        check(hip().dnn_hip_decode(self.ptr, _ip(feed), feed.shape[0], _ip(nf) if nf is not None else None,
                                   n_steps, eos, _ip(ids), _fp(lg) if want_logits else None, C.byref(done)))
        d = done.value
        return ids[:d], (lg[:d] if want_logits else None)

    def prefill(self, ids=None, n_ids=None, embeds=None, mode=0, prefix_len=0, want_logits=False):
        """Multi-token prefill.  ids: [B][n_max] ints (or None), n_ids: [B] or None,
        embeds: [B][n_embed][D] floats or None.  Returns (next_ids [B], logits [B][V] or None)."""
        B = self.B
        if ids is None:
            ids_a, n_max = None, 0
        else:
            ids_a = np.ascontiguousarray(ids, dtype=np.int32).reshape(B, -1)
            n_max = ids_a.shape[1]
        nid = None if n_ids is None else np.ascontiguousarray(n_ids, dtype=np.int32)
        if embeds is None:
            emb, n_emb = None, 0
        else:
            emb = np.ascontiguousarray(embeds, dtype=np.float32).reshape(B, -1, self.m.D)
            n_emb = emb.shape[1]
        nxt = np.zeros(B, dtype=np.int32)
        lg = np.zeros((B, self.m.V), dtype=np.float32) if want_logits else None
        check(hip().dnn_hip_prefill(self.ptr, _fp(emb) if emb is not None else None, n_emb,
                                    _ip(ids_a) if ids_a is not None else None, n_max,
                                    _ip(nid) if nid is not None else None, mode, prefix_len, _ip(nxt),
                                    _fp(lg) if want_logits else None))
        return nxt, lg

    def block_forward(self, layer, x, pos0, mode=0, prefix_len=0):
        """x [B][n_new][D] -> y [B][n_new][D] through one block at positions pos0.."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros_like(x)
        check(hip().dnn_hip_block_forward(self.ptr, layer, _fp(x), x.shape[1], pos0, mode, prefix_len, _fp(y)))
        return y

    def head_forward(self, x, norm=True):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.m.D)
        lg = np.zeros((x.shape[0], self.m.V), dtype=np.float32)
        check(hip().dnn_hip_head_forward(self.ptr, _fp(x), x.shape[0], 1 if norm else 0, _fp(lg)))
        return lg

    def embed(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        out = np.zeros((len(ids), self.m.D), dtype=np.float32)
        check(hip().dnn_hip_embed(self.ptr, _ip(ids), len(ids), _fp(out)))
        return out

    def rms_norm(self, x, gamma, eps=1e-5):
        """rms_norm of the rows of x [n][d] with gamma [d], on the device."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        g = np.ascontiguousarray(gamma, dtype=np.float32)
        y = np.zeros_like(x)
        d = x.shape[-1]
        check(hip().dnn_hip_rms_norm(self.ptr, _fp(x), _fp(g), x.size // d, d, C.c_float(eps), _fp(y)))
        return y

    def cache_read(self, layer, which, length):
        out = np.zeros((self.B, self.m.H, length, 64), dtype=np.float32)
        check(hip().dnn_hip_cache_read(self.ptr, layer, which, length, _fp(out)))
        return out

    def last_ms(self):
        ms = C.c_float()
        check(hip().dnn_hip_session_last_ms(self.ptr, C.byref(ms)))
        return ms.value

    def lengths(self):
        out = np.zeros(self.B, dtype=np.int32)
        check(hip().dnn_hip_session_lengths(self.ptr, _ip(out)))
        return out

    def reset(self):
        check(hip().dnn_hip_session_reset(self.ptr))

    def close(self):
        if getattr(self, "ptr", None):
            hip().dnn_hip_session_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
