"""dnn_hip_decode_static -- the decode entry point that allocates nothing (its
scratch is a fixed device array of the library; the caller owns every other
buffer) -- against dnn_hip_decode on the same inputs, through the C-ABI.

Two calls in a row: two rows with ragged prompts and 30 steps, then one row
with a shorter prompt and 12 steps (a smaller input: the shared scratch array
still holds the first call's values).  Both entry points run the same kernel
with the same launch shape, so the tokens, logits and row lengths must be
identical bit for bit.  A model whose exchange arena would not fit the array
is refused before any device work.
"""
import ctypes as C

import numpy as np
import pytest

import dnn_amd as A
import oracle_lib as O

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class Rt:
    """The caller's own device buffers (hipMalloc through the HIP runtime the
    library is linked against)."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.bufs = []

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), max(nbytes, 4)) == 0
        self.bufs.append(p)
        return p

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        assert self.rt.hipMemcpy(p, a.ctypes.data, a.nbytes, H2D) == 0
        return p

    def get(self, p, shape, dtype):
        out = np.zeros(shape, dtype=dtype)
        assert self.rt.hipMemcpy(out.ctypes.data, p, out.nbytes, D2H) == 0
        return out

    def free(self):
        assert self.rt.hipDeviceSynchronize() == 0
        for p in self.bufs:
            self.rt.hipFree(p)
        self.bufs = []


def lib():
    L = A.hip()
    L.dnn_hip_kv_floats.argtypes = [C.c_void_p, C.c_int, C.c_int]
    L.dnn_hip_kv_floats.restype = C.c_size_t
    L.dnn_hip_decode_static.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                        C.c_void_p, C.c_void_p]
    L.dnn_hip_decode_static_status.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]
    return L


def static_decode(rt, hm, feed, n_feed, steps, max_seq):
    """One dnn_hip_decode_static call on fresh caller buffers (empty rows)."""
    L = lib()
    feed = np.ascontiguousarray(feed, dtype=np.int32)
    B = feed.shape[1]
    kvf = L.dnn_hip_kv_floats(hm.ptr, B, max_seq)
    assert kvf > 0
    kc, vc = rt.alloc(kvf * 4), rt.alloc(kvf * 4)
    pos = rt.put(np.zeros(B, np.int32))
    d_feed, d_nf = rt.put(feed), rt.put(np.asarray(n_feed, np.int32))
    ids = rt.alloc(steps * B * 4)
    lg = rt.alloc(steps * B * hm.V * 4)
    A.check(L.dnn_hip_decode_static(hm.ptr, B, max_seq, kc, vc, pos, d_feed, d_nf, steps, -1, steps, ids, lg, None))
    done, err = C.c_int(), C.c_int()
    A.check(L.dnn_hip_decode_static_status(None, C.byref(done), C.byref(err)))
    assert done.value == steps and err.value == 0
    return (rt.get(ids, (steps, B), np.int32), rt.get(lg, (steps, B, hm.V), np.float32),
            rt.get(pos, (B,), np.int32))


def test_static_decode_equals_session_decode():
    m = O.Model(128, 256, 4, 4, 683, 64, seed=11, init="gpt2")
    hm = A.HipModel(m.V, m.D, m.L, m.H, m.F, m.params(), rope=m.rope_tables())
    rng = np.random.default_rng(707)
    rt = Rt()
    try:
        cases = [(rng.integers(0, 128, size=(6, 2)), np.array([6, 3]), 30),
                 (rng.integers(0, 128, size=(4, 1)), np.array([4]), 12)]
        for i, (feed, nf, steps) in enumerate(cases):
            print("static decode call %d: batch %d, %d steps" % (i, feed.shape[1], steps), flush=True)
            s = A.HipSession(hm, feed.shape[1], 64)
            want_ids, want_lg = s.decode(feed, steps, n_feed=nf, want_logits=True)
            assert s.kernel() == 3
            ids, lg, pos = static_decode(rt, hm, feed, nf, steps, 64)
            assert np.array_equal(ids, want_ids), "call %d: ids" % i
            assert np.array_equal(lg.view(np.uint32), want_lg.view(np.uint32)), "call %d: logits" % i
            assert list(pos) == list(s.lengths()) == [steps] * feed.shape[1]
            s.close()
    finally:
        rt.free()


def test_static_decode_refuses_oversized_scratch():
    """40 layers of d_ffn 2048 at batch 8 need more exchange pairs than the
    static array holds: refused with DNN_HIP_EINVAL, nothing launched."""
    V, D, L, H, F = 128, 256, 40, 4, 2048
    rng = np.random.default_rng(9)
    shapes = [(V, D)] + [s for _ in range(L) for s in ((D, 3 * D), (3 * D,), (D, D), (D,), (D,), (D,), (D, F), (F,),
                                                        (D, F), (F,), (F, D), (D,))] + [(D,), (V,)]
    params = [(rng.standard_normal(sh) * 0.02).astype(np.float32) for sh in shapes]
    hm = A.HipModel(V, D, L, H, F, params)
    Lb = lib()
    rt = Rt()
    try:
        p = rt.alloc(64)
        rc = Lb.dnn_hip_decode_static(hm.ptr, 8, 32, p, p, p, p, p, 4, -1, 4, p, None, None)
        assert rc == -1, rc
        assert b"static arena" in Lb.dnn_hip_last_error()
    finally:
        rt.free()
