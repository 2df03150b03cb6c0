"""The reference's layer-level API on the device: transformer_block_forward_cached(_ex),
rms_norm_forward, decoder_lm_lm_head_forward, decoder_lm_token_embeds / forward,
tensor_cat and kv_cache_get_K/V, driven from C the way gpt.c:306-375 and
vlm.c:497-565 drive them (tests/c/block_main.c), and the C-ABI calls under them
(dnn_hip_block_forward, dnn_hip_head_forward, dnn_hip_embed, dnn_hip_rms_norm,
dnn_hip_cache_read) from Python against the oracle.

Bars: ids identical to the reference's fixtures; logits within max-abs 1e-3 and
relative 1e-4 per row; hidden states and cached K/V
rows within 1e-4 of the oracle's."""
import json
import os
import subprocess

import numpy as np
import pytest

import dnn_amd as A
import oracle_lib as O
from golden_util import binf
from test_parity_gpu import assert_logits_close, hip_model

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def block_main(built, tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("c") / "block_main")
    libdir = os.path.join(ROOT, "dnn.c_amd", "lib")
    subprocess.check_call(["gcc", "-std=gnu11", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "c", "block_main.c"), "-o", exe,
                           "-L" + libdir, "-ldnn_amd", "-Wl,-rpath," + libdir, "-lm"])
    return exe


def run(exe, mode, out):
    print("block_main", mode, flush=True)
    r = json.loads(subprocess.check_output([exe, mode, str(out)], text=True, timeout=300))
    return r, lambda name, cols: np.fromfile(os.path.join(out, name + ".f32"), dtype=np.float32).reshape(-1, cols)


def test_c_block_api_c1(block_main, golden, tmp_path):
    """C1 through the per-layer API: the token-by-token run (the reference's
    manual generate loop), the multi-token cached prefill of the prompt and
    decoder_lm_forward over 24 ids, each against the reference's fixtures; the
    last layer's cache as kv_cache_get_K/V return it, against the oracle."""
    r, load = run(block_main, "c1", tmp_path)
    assert r["c1_tokens"] == golden["c1_tokens"]
    assert_logits_close(load("c1_logits", 128), binf("c1_logits.f32", 128), "token-by-token")
    assert r["c1_prefill_tokens"] == golden["c1_prefill_tokens"]
    assert_logits_close(load("c1_prefill_logits", 128), binf("c1_prefill_logits.f32", 128), "prefill")
    assert_logits_close(load("c1_full24_logits", 128), binf("c1_full24_logits.f32", 128), "full forward")
    n = len(golden["c1_tokens"]) - 1            # every id but the last was fed
    assert r["c1_cache_shape"] == [1, 4, n, 64]
    m = O.Model(128, 256, 4, 4, 683, 256, seed=1)
    st = O.State(m, 256)
    for t in golden["c1_tokens"][:n]:
        st.forward(O.embed(m, np.array([t], dtype=np.int32)))
    for which, name in ((0, "c1_K3"), (1, "c1_V3")):
        got = load(name, 64).reshape(4, n, 64)
        np.testing.assert_allclose(got, st.cache(3, which, n), atol=1e-4, rtol=0, err_msg=name)


def test_c_block_api_prefix_lm(block_main, golden, tmp_path):
    """The VLM shape: 12 prefix rows ++ 4 text ids (tensor_cat), one PREFIX_LM
    cached_ex pass per layer, then 6 causal decode steps."""
    r, load = run(block_main, "vlm", tmp_path)
    assert r["vlm_tokens"] == golden["vlm_tokens"]
    assert_logits_close(load("vlm_logits", 96), binf("vlm_logits.f32", 96), "prefix-LM")


@pytest.fixture(scope="module")
def c1g():
    m = O.Model(128, 256, 4, 4, 683, 256, seed=11, init="gpt2")
    return m, hip_model(m)


@pytest.mark.parametrize("B,N", [(1, 1), (3, 5), (2, 70)])
def test_block_forward_rows_vs_oracle(c1g, B, N):
    """dnn_hip_block_forward over every layer for B rows of N new positions,
    then 2 single-position steps, each row against its own oracle sequence;
    dnn_hip_head_forward (with and without the final norm) on the result and
    dnn_hip_cache_read of every layer."""
    m, hm = c1g
    print("block_forward B=%d N=%d" % (B, N), flush=True)
    rng = np.random.default_rng(B * 100 + N)
    ids = rng.integers(0, 128, size=(B, N + 2)).astype(np.int32)
    s = A.HipSession(hm, B, N + 2)
    st = [O.State(m, N + 2) for _ in range(B)]
    pos = 0
    for n in (N, 1, 1):
        x = s.embed(ids[:, pos:pos + n]).reshape(B, n, m.D)
        for b in range(B):
            np.testing.assert_array_equal(x[b], O.embed(m, ids[b, pos:pos + n]))
        for layer in range(m.L):
            x = s.block_forward(layer, x, pos)
        want = np.stack([st[b].forward(O.embed(m, ids[b, pos:pos + n])) for b in range(B)])
        np.testing.assert_allclose(x, want, atol=1e-4, rtol=0)
        assert_logits_close(s.head_forward(x), np.concatenate([O.head(m, w) for w in want]), "head n=%d" % n)
        pos += n
    assert list(s.lengths()) == [0] * B        # block calls leave the session's own lengths alone
    for layer in range(m.L):
        for which in (0, 1):
            got = s.cache_read(layer, which, pos)
            for b in range(B):
                np.testing.assert_allclose(got[b], st[b].cache(layer, which, pos), atol=1e-4, rtol=0)
    # head without the final norm: rms_norm(x) first, with the final gamma
    g = m.params()[-2]
    xn = s.rms_norm(x.reshape(-1, m.D), g)
    assert_logits_close(s.head_forward(xn, norm=False), s.head_forward(x), "norm split")


def test_rms_norm_rows_vs_oracle():
    """dnn_hip_rms_norm against the oracle's tensor_rms_norm (norm.c:404-495) on
    rows of d = 96 and 256 with a non-trivial gamma."""
    m = O.Model(128, 256, 1, 4, 64, 16, seed=3)
    s = A.HipSession(hip_model(m), 1, 8)
    rng = np.random.default_rng(5)
    for d in (96, 256):
        x = rng.standard_normal((7, d)).astype(np.float32) * 3
        g = rng.standard_normal(d).astype(np.float32)
        want = np.zeros_like(x)
        O.lib().orc_rms_norm(O.fp(x), O.fp(g), O.fp(want), 7, d, np.float32(1e-5))
        np.testing.assert_allclose(s.rms_norm(x, g), want, atol=1e-5, rtol=1e-5)


def test_block_api_errors(c1g):
    m, hm = c1g
    s = A.HipSession(hm, 2, 8)
    x = np.zeros((2, 4, m.D), dtype=np.float32)
    with pytest.raises(A.HipError, match="max_seq"):
        s.block_forward(0, x, 6)
    with pytest.raises(A.HipError, match="prefix-LM"):
        s.block_forward(0, x, 2, mode=1, prefix_len=2)
    with pytest.raises(A.HipError, match="layer"):
        s.block_forward(m.L, x, 0)
    with pytest.raises(A.HipError, match="outside"):
        s.embed(np.array([128], dtype=np.int32))
