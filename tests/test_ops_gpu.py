"""The reference's op- and layer-level API on the device, driven from C.

tests/c/ops_main.c calls only functions the reference's headers declare
(tensor_matmul_add, tensor_add, tensor_swiglu, tensor_embedding,
tensor_rms_norm, tensor_rope, tensor_split_qkv_heads, tensor_merge_heads,
tensor_split_heads, linear_forward, swiglu_ffn_forward,
transformer_block_forward(_ex), decoder_lm_hidden_from_embeds(_ex)) on inputs
drawn from the seeded default stream.  tests/golden/make_golden.sh built the
same file against the reference and wrote its outputs to
tests/golden/data/ops/; here it is built against include/dnn + libdnn_amd.so.

Bars: the matmul (k summed in order, bias last, no FMA contraction), the
elementwise add, RoPE, the gather and the layout transforms are compared bit
for bit; SwiGLU (device expf), rms_norm (tree sum of squares) and the layers
built on them within max |d| <= 1e-5 * max(1, max |ref|), and the block and
hidden-state forwards (attention on MFMA-free device kernels, other summation
order) within 1e-4 of the same scale.  Rows past a seq_lens length, which the
reference leaves uncomputed, are checked to be zero here.
"""
import os
import subprocess

import numpy as np
import pytest

from golden_util import DATA

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

EXACT = ["mm2", "mm2t", "mm3", "mm3b", "add_same", "add_bias", "add_bcast", "embedding", "rope", "split_q",
         "split_k", "split_v", "merge", "split_heads", "linear"]
CLOSE = {"swiglu": 1e-5, "rms_w": 1e-5, "rms_nw": 1e-5, "ffn": 1e-5, "block_causal": 1e-4, "block_prefix": 1e-4,
         "hidden": 1e-4, "hidden_prefix": 1e-4}


@pytest.fixture(scope="module")
def ops_out(built, tmp_path_factory):
    d = tmp_path_factory.mktemp("ops")
    exe = str(d / "ops_main")
    libdir = os.path.join(ROOT, "dnn.c_amd", "lib")
    subprocess.check_call(["gcc", "-std=gnu11", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include", "dnn"),
                           os.path.join(ROOT, "tests", "c", "ops_main.c"), "-o", exe,
                           "-L" + libdir, "-ldnn_amd", "-Wl,-rpath," + libdir, "-lm"])
    print("ops_main", flush=True)
    out = subprocess.check_output([exe, str(d)], text=True, timeout=120)
    assert out.strip() == "ok"
    return str(d)


def load(d, name):
    return np.fromfile(os.path.join(d, name + ".f32"), dtype=np.float32)


@pytest.mark.parametrize("name", EXACT)
def test_op_bits_equal_reference(ops_out, name):
    got, want = load(ops_out, name), load(os.path.join(DATA, "ops"), name)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        "%s: %d of %d values differ" % (name, int((got != want).sum()), got.size)


@pytest.mark.parametrize("name", sorted(CLOSE))
def test_op_close_to_reference(ops_out, name):
    got, want = load(ops_out, name).astype(np.float64), load(os.path.join(DATA, "ops"), name).astype(np.float64)
    assert got.shape == want.shape
    err = np.abs(got - want).max()
    bar = CLOSE[name] * max(1.0, np.abs(want).max())
    assert err <= bar, "%s: max |d| %.3g > %.3g" % (name, err, bar)


@pytest.mark.parametrize("name", ["block_lens", "hidden_lens"])
def test_seq_lens_rows(ops_out, name):
    """Batch row 0 runs all 9 rows, row 1 its first 6 (seq_lens {9, 6})."""
    got = load(ops_out, name).reshape(2, 9, 128).astype(np.float64)
    want = load(os.path.join(DATA, "ops"), name).reshape(2, 9, 128).astype(np.float64)
    for b, n in ((0, 9), (1, 6)):
        err = np.abs(got[b, :n] - want[b, :n]).max()
        assert err <= 1e-4 * max(1.0, np.abs(want[b, :n]).max()), "%s row %d: %.3g" % (name, b, err)
    assert not got[1, 6:].any()
