"""Pins the CPU oracle (oracle/dnn_oracle.c) to the reference.

Every expected value below was written by the real reference (masc-it/dnn.c
compiled from its sources by oracle/Makefile, run by tests/golden/gen_golden.c).
The oracle must reproduce it bit for bit: RNG streams, create-time and
GPT-2-style initialisation, RoPE tables, each single op, the cached block over a
whole greedy run (C1 shape, two inits), multi-token cached prefill, prefix-LM
prefill, and the no-cache full forward.  A plausible slip in the restatement (a
dropped bias, a swapped rope sign, Q/K column blocks exchanged, a different
summation order) changes the bits and fails here.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from golden_util import binf, f32, same_bits


@pytest.fixture(scope="module")
def L(built):
    return O.lib()


def test_rng_streams_match_reference(L, golden):
    for seed in (0, 1, 42, 12345):
        r = O.Rng()
        L.orc_rng_seed(C.byref(r), seed)
        assert ["%016x" % r.s[0], "%016x" % r.s[1]] == golden["rng_%d_state" % seed]
        u = np.array([L.orc_rng_uniform(C.byref(r)) for _ in range(8)], dtype=np.float32)
        n = np.array([L.orc_rng_normal(C.byref(r)) for _ in range(8)], dtype=np.float32)
        i = [L.orc_rng_uniform_int(C.byref(r), 8192) for _ in range(8)]
        j = [L.orc_rng_uniform_int(C.byref(r), 49) for _ in range(8)]
        assert same_bits(u, f32(golden, "rng_%d_uniform" % seed))
        assert same_bits(n, f32(golden, "rng_%d_normal" % seed))
        assert i == golden["rng_%d_int8192" % seed]
        assert j == golden["rng_%d_int49" % seed]


def test_splitmix_closed_form(L):
    """SplitMix64's first output for seed 0 is a published constant."""
    r = O.Rng()
    L.orc_rng_seed(C.byref(r), 0)
    assert r.s[0] == 0xE220A8397B1DCDAF


def test_matmul_add_both_layouts(L, golden):
    a = f32(golden, "op_mm_a").reshape(6, 37)
    w = f32(golden, "op_mm_w").reshape(37, 53)
    wt = f32(golden, "op_mm_wt").reshape(53, 37)
    b = f32(golden, "op_mm_b")
    y = np.zeros((6, 53), np.float32)
    L.orc_matmul_add(O.fp(a), O.fp(w), O.fp(b), O.fp(y), 6, 37, 53, 0)
    assert same_bits(y, f32(golden, "op_mm_y").reshape(6, 53))
    L.orc_matmul_add(O.fp(a), O.fp(wt), O.fp(b), O.fp(y), 6, 37, 53, 1)
    assert same_bits(y, f32(golden, "op_mm_yt").reshape(6, 53))
    # and the mathematics: fp64 product agrees to float rounding
    ref = a.astype(np.float64) @ w.astype(np.float64) + b
    L.orc_matmul_add(O.fp(a), O.fp(w), O.fp(b), O.fp(y), 6, 37, 53, 0)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("d", [768, 683])
def test_rms_norm(L, golden, d):
    x = f32(golden, "op_rms%d_x" % d).reshape(3, d)
    g = f32(golden, "op_rms%d_g" % d)
    y = np.zeros_like(x)
    L.orc_rms_norm(O.fp(x), O.fp(g), O.fp(y), 3, d, np.float32(1e-5))
    assert same_bits(y, f32(golden, "op_rms%d_y" % d).reshape(3, d))
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * g
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_rope_table_and_rotation(L, golden):
    m = O.Model(128, 128, 1, 2, 64, 1088, seed=0, init="create")
    cos, sin = m.rope_tables()
    assert O.fnv(cos) == golden["rope_cos_hash"]
    assert O.fnv(sin) == golden["rope_sin_hash"]
    assert same_bits(cos[1000], f32(golden, "rope_cos_row1000"))
    x = f32(golden, "op_rope_x").reshape(2, 5, 64).copy()
    for h in range(2):
        row = np.ascontiguousarray(x[h])
        L.orc_rope_rows(O.fp(row), 5, 64, O.fp(np.ascontiguousarray(cos[7:12])), O.fp(np.ascontiguousarray(sin[7:12])))
        x[h] = row
    assert same_bits(x.reshape(-1), f32(golden, "op_rope_y"))
    # a rotation keeps each pair's norm
    x0 = f32(golden, "op_rope_x").reshape(-1, 2).astype(np.float64)
    assert np.allclose(np.hypot(*x0.T), np.hypot(*x.reshape(-1, 2).astype(np.float64).T), rtol=1e-6)


def test_swiglu(L, golden):
    g, u = f32(golden, "op_swiglu_g"), f32(golden, "op_swiglu_u")
    y = np.zeros_like(g)
    L.orc_swiglu(O.fp(g), O.fp(u), O.fp(y), len(g))
    assert same_bits(y, f32(golden, "op_swiglu_y"))
    g64 = g.astype(np.float64)
    assert np.allclose(y, g64 / (1 + np.exp(-g64)) * u, rtol=1e-5, atol=1e-6)


def test_init_hashes(golden):
    assert [O.fnv(p) for p in O.Model(128, 256, 4, 4, 683, 256, seed=1).params()] == golden["c1_params"]
    assert [O.fnv(p) for p in O.Model(128, 256, 4, 4, 683, 256, seed=7, init="create").params()] == golden["c1_create_params"]
    assert [O.fnv(p) for p in O.Model(128, 256, 4, 4, 683, 256, seed=7, init="gpt2").params()] == golden["c1_gpt2_params"]
    assert [O.fnv(p) for p in O.Model(128, 256, 4, 4, 683, 256, seed=11, init="gpt2").params()] == golden["c1g_params"]


@pytest.mark.parametrize("tag,seed,init,pseed", [("c1", 1, "synthetic", 101), ("c1g", 11, "gpt2", 111)])
def test_greedy_run_bit_exact(golden, tag, seed, init, pseed):
    """240 greedy steps of the C1 shape: every token and every logit bit."""
    m = O.Model(128, 256, 4, 4, 683, 256, seed=seed, init=init)
    prompt = O.prompt_ids(pseed, 128, 16)
    assert list(prompt) == golden[tag + "_prompt"]
    toks, lg = m.generate(prompt, 240, want_logits=True)
    assert list(toks) == golden[tag + "_tokens"]
    assert same_bits(lg, binf(tag + "_logits.f32", 128))


def test_generate_api_and_nocache_agree_with_manual_loop(golden):
    """The reference's own decoder_lm_generate, cached and not, gave the same ids
    as the per-layer loop the fixtures record (cached == non-cached)."""
    assert golden["c1_generate_tokens"] == golden["c1_tokens"]
    assert golden["c1_nocache_tokens"] == golden["c1_tokens"][: len(golden["c1_nocache_tokens"])]


def test_full_forward_equals_reference(golden):
    m = O.Model(128, 256, 4, 4, 683, 256, seed=1)
    lg = m.forward_full(np.array(golden["c1_tokens"][:24]))
    assert same_bits(lg, binf("c1_full24_logits.f32", 128))


def test_multi_token_prefill(golden):
    """One cached call over the whole prompt, then 8 single-token steps."""
    m = O.Model(128, 256, 4, 4, 683, 256, seed=1)
    st = O.State(m, 64)
    prompt = np.array(golden["c1_prompt"], dtype=np.int32)
    h = st.forward(O.embed(m, prompt))
    lg = [O.head(m, h[-1:])[0]]
    ids = [O.lib().orc_argmax(O.fp(lg[0]), 128)]
    for _ in range(8):
        h = st.forward(O.embed(m, np.array(ids[-1:], dtype=np.int32)))
        lg.append(O.head(m, h)[0])
        ids.append(O.lib().orc_argmax(O.fp(lg[-1]), 128))
    assert ids == golden["c1_prefill_tokens"]
    assert same_bits(np.array(lg), binf("c1_prefill_logits.f32", 128))


def test_prefix_lm_prefill(golden):
    """VLM shape: 12 bidirectional prefix rows + 4 text rows in one prefix-LM pass,
    then 6 causal decode steps."""
    m = O.Model(96, 128, 2, 2, 256, 64, seed=5)
    assert [O.fnv(p) for p in m.params()] == golden["vlm_params"]
    prefix = f32(golden, "vlm_prefix").reshape(12, 128)
    text = np.array(golden["vlm_text"], dtype=np.int32)
    st = O.State(m, 22)
    x = np.concatenate([prefix, O.embed(m, text)])
    h = st.forward(x, mode=1, prefix_len=12)
    rows = [O.head(m, h)]
    ids = [int(np.argmax(rows[0][-1]))]
    for _ in range(6):
        h = st.forward(O.embed(m, np.array(ids[-1:], dtype=np.int32)))
        rows.append(O.head(m, h))
        ids.append(int(np.argmax(rows[-1][0])))
    assert ids == golden["vlm_tokens"]
    assert same_bits(np.concatenate(rows), binf("vlm_logits.f32", 96))


def test_batch_rows_match_reference(golden):
    """Six independent B=1 runs with prompt lengths 4..16."""
    m = O.Model(128, 256, 4, 4, 683, 256, seed=1)
    lens = golden["c1_batch_lens"]
    prompts = np.array(golden["c1_batch_prompts"], dtype=np.int32).reshape(6, 16)
    want = np.array(golden["c1_batch_tokens"]).reshape(6, 48)
    for b in range(6):
        got = m.generate(prompts[b, : lens[b]], 32)
        assert list(got) == [t for t in want[b] if t >= 0]


def test_c2_first_steps_and_hashes(golden):
    """C2 (the headline config): weights, prompt and the first 4 steps' logits."""
    m = O.Model(8192, 768, 12, 12, 2048, 1088, seed=2)
    assert [O.fnv(p) for p in m.params()] == golden["c2_params"]
    prompt = O.prompt_ids(102, 8192, 32)
    assert list(prompt) == golden["c2_prompt"]
    toks, lg = m.generate(prompt, 4, want_logits=True)
    assert same_bits(lg, binf("c2_logits4.f32", 8192))
    assert list(toks) == golden["c2_tokens"][:36]


def test_cache_rows_closed_form():
    """orc_state_kv hands back layer 0's cached K/V rows as the closed form
    fixes them: V = rms_norm(x) Wv + bv, K = RoPE_p(rms_norm(x) Wk + bk) at
    each position p (transformer.c:223-247; fp64 here, so a tolerance), in
    kv_cache_get_K/V order [H][len][dk]; and rows once written never change."""
    m = O.Model(128, 256, 4, 4, 683, 64, seed=1)
    p = m.params()
    D, H, dk = 256, 4, 64
    wqkv = p[1].reshape(D, 3 * D).astype(np.float64)
    bqkv = p[2].astype(np.float64)
    g = p[5].astype(np.float64)
    cos, sin = m.rope_tables()
    ids = np.array([5, 77, 3, 120, 64], dtype=np.int32)
    x = O.embed(m, ids).astype(np.float64)
    xn = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-5) * g
    qkv = xn @ wqkv + bqkv
    k = qkv[:, D:2 * D].reshape(5, H, dk)
    v = qkv[:, 2 * D:].reshape(5, H, dk)
    c, s = cos[:5, None, :], sin[:5, None, :]
    e, o = k[..., 0::2].copy(), k[..., 1::2].copy()
    k[..., 0::2], k[..., 1::2] = e * c - o * s, e * s + o * c
    st = O.State(m, 64)
    st.forward(O.embed(m, ids[:3]))
    k3 = st.cache(0, 0, 3)
    st.forward(O.embed(m, ids[3:]))
    got_k, got_v = st.cache(0, 0, 5), st.cache(0, 1, 5)
    assert got_k.shape == (H, 5, dk)
    np.testing.assert_allclose(got_k, k.transpose(1, 0, 2), atol=2e-5)
    np.testing.assert_allclose(got_v, v.transpose(1, 0, 2), atol=2e-5)
    assert same_bits(got_k[:, :3], k3)
