"""GPU parity of the batched engine (more than 8 rows, bf16 weights, multi-token
prefill) against the oracle and the reference's fixtures.

Bars: greedy tokens identical; logits within
max-abs 1e-3 and relative 1e-4 (max |dlogit| / max |logit| per row).  The bf16
variant is checked against the oracle run on the same bf16-rounded weights
(W16A32), to the same bar: only the summation order differs.
"""
import numpy as np
import pytest

import dnn_amd as A
import oracle_lib as O
from golden_util import binf
from test_parity_gpu import assert_logits_close, hip_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def c1g():
    return O.Model(128, 256, 4, 4, 683, 256, seed=11, init="gpt2")


# the GEMMs' row tiles per workgroup away from the defaults: two (QKV, gate/up),
# all rows (down), one (lm_head)
TILES = {"DNN_HIP_QKV_MT": "2", "DNN_HIP_GU_MT": "2", "DNN_HIP_DOWN_MT": "0", "DNN_HIP_HEAD_MT": "1"}


@pytest.mark.parametrize("B,splits,tiles", [(16, None, False), (33, None, False), (64, None, False),
                                            (16, 3, False), (12, 8, False), (64, None, True), (48, None, True)])
def test_engine_rows_match_independent_runs(c1g, B, splits, tiles, monkeypatch):
    """Every row of a batched decode (the engine: more than 8 rows) equals its
    own B=1 oracle run; rows switch from prompt to greedy at different steps.
    With `splits` (DNN_HIP_ATT_SPLITS) each head's keys are split over that
    many workgroups and merged by the last one to arrive; with `tiles` the
    GEMMs take other row tiles per workgroup than the defaults."""
    if splits:
        monkeypatch.setenv("DNN_HIP_ATT_SPLITS", str(splits))
    if tiles:
        for k, v in TILES.items():
            monkeypatch.setenv(k, v)
    hm = hip_model(c1g)
    rng = np.random.default_rng(100 + B)
    lens = rng.integers(1, 9, size=B).astype(np.int32)
    feed = rng.integers(0, 128, size=(8, B)).astype(np.int32)
    steps = 40
    print("engine rows B=%d splits=%s tiles=%s" % (B, splits, tiles), flush=True)
    s = A.HipSession(hm, B, 72)
    ids, lg = s.decode(feed, steps, n_feed=lens, want_logits=True)
    assert s.kernel() == 6
    assert s.att_splits() == (splits or 1)
    for b in range(B):
        want, wlg = c1g.generate(feed[: lens[b], b], steps - lens[b] + 1, eos=-1, want_logits=True)
        got = list(feed[: lens[b], b]) + list(ids[lens[b] - 1:, b])
        assert got == list(want), "row %d" % b
        assert_logits_close(lg[lens[b] - 1:, b], wlg, "row %d" % b)
    assert list(s.lengths()) == [steps] * B
    # a second call continues every row from its cached length
    ids2, _ = s.decode(ids[-1:], 8)
    for b in range(B):
        want = c1g.generate(feed[: lens[b], b], steps - lens[b] + 9, eos=-1)
        assert list(ids2[:, b]) == list(want[steps + 1:steps + 9]), "row %d, second call" % b


def test_engine_without_graph_equals_graph(c1g, monkeypatch):
    """DNN_HIP_ENGINE_GRAPH=0 launches each step's kernels directly instead of
    replaying the captured step graph: the same tokens and logits, bit for bit."""
    hm = hip_model(c1g)
    rng = np.random.default_rng(77)
    B = 16
    lens = rng.integers(1, 9, size=B).astype(np.int32)
    feed = rng.integers(0, 128, size=(8, B)).astype(np.int32)
    s = A.HipSession(hm, B, 48)
    ids_g, lg_g = s.decode(feed, 30, n_feed=lens, want_logits=True)
    monkeypatch.setenv("DNN_HIP_ENGINE_GRAPH", "0")
    s2 = A.HipSession(hm, B, 48)
    ids_e, lg_e = s2.decode(feed, 30, n_feed=lens, want_logits=True)
    assert s.kernel() == 6 and s2.kernel() == 6
    assert np.array_equal(ids_g, ids_e)
    assert np.array_equal(lg_g.view(np.uint32), lg_e.view(np.uint32))


def test_engine_c2_tokens_and_logits_match_reference(golden, monkeypatch):
    """The C2 model on the engine (one row, forced): the reference's own greedy
    tokens and its logits of the first four generated steps."""
    m = O.Model(8192, 768, 12, 12, 2048, 1088, seed=2)
    hm = hip_model(m)
    monkeypatch.setenv("DNN_HIP_DECODE_KERNEL", "6")
    toks = golden["c2_tokens"]
    s = A.HipSession(hm, 1, 200)
    ids, _ = s.decode(np.array(toks[:32], dtype=np.int32), 160, n_feed=np.array([32], np.int32))
    assert s.kernel() == 6
    assert list(ids[31:, 0]) == toks[32:161]
    s2 = A.HipSession(hm, 1, 64)
    _, lg = s2.decode(np.array(toks[:35], dtype=np.int32), 35, want_logits=True)
    assert_logits_close(lg[31:, 0], binf("c2_logits4.f32", 8192), "c2 first 4 steps (engine)")


def test_engine_equals_persistent_kernel_c2_b8(golden, monkeypatch):
    """Eight C2 rows: the engine's tokens equal the persistent kernel's and its
    logits agree within the bar (different summation order)."""
    m = O.Model(8192, 768, 12, 12, 2048, 1088, seed=2)
    hm = hip_model(m)
    rng = np.random.default_rng(8)
    feed = rng.integers(0, 8192, size=(6, 8)).astype(np.int32)
    monkeypatch.setenv("DNN_HIP_DECODE_KERNEL", "3")
    s3 = A.HipSession(hm, 8, 64)
    ids3, lg3 = s3.decode(feed, 40, want_logits=True)
    monkeypatch.setenv("DNN_HIP_DECODE_KERNEL", "6")
    s6 = A.HipSession(hm, 8, 64)
    ids6, lg6 = s6.decode(feed, 40, want_logits=True)
    assert s3.kernel() == 3 and s6.kernel() == 6
    assert np.array_equal(ids3, ids6)
    for b in range(8):
        assert_logits_close(lg6[:, b], lg3[:, b], "row %d" % b)


def test_engine_long_history_splits(monkeypatch):
    """Six rows past 1,024 cached keys: the engine splits each head's keys over
    two workgroups (at most two 64-key chunks per wavefront of eight) and the
    tokens and logits still follow the oracle's generation from each prompt."""
    monkeypatch.delenv("DNN_HIP_ATT_SPLITS", raising=False)
    m = O.Model(128, 256, 4, 4, 683, 1100, seed=11, init="gpt2")
    hm = hip_model(m)
    B, steps = 6, 12
    rng = np.random.default_rng(61)
    n = rng.integers(1030, 1061, size=B).astype(np.int32)
    ids = rng.integers(0, 128, size=(B, int(n.max()))).astype(np.int32)
    print("engine long history n=%s" % list(n), flush=True)
    s = A.HipSession(hm, B, 1100)
    nxt, _ = s.prefill(ids=ids, n_ids=n)
    out, lg = s.decode(nxt, steps, want_logits=True)
    assert s.kernel() == 6 and s.att_splits() == 2
    for b in range(B):
        want, wlg = m.generate(ids[b, : n[b]], steps + 1, eos=-1, want_logits=True)
        assert [int(nxt[b])] + list(out[:, b]) == list(want[n[b]:]), "row %d" % b
        assert_logits_close(lg[:, b], wlg[1:], "row %d" % b)


@pytest.mark.parametrize("B", [1, 5, 12])
def test_prefill_causal_matches_cached_forward(c1g, B):
    """dnn_hip_prefill over ragged prompts (some longer than one 64-row tile)
    equals the oracle's multi-token cached forward (transformer.c:211-416) at
    each row's last position; decoding on from there equals the oracle's
    generation from the same prompt."""
    hm = hip_model(c1g)
    rng = np.random.default_rng(200 + B)
    n = rng.integers(1, 150, size=B).astype(np.int32)
    ids = rng.integers(0, 128, size=(B, int(n.max()))).astype(np.int32)
    print("prefill causal B=%d n=%s" % (B, list(n)), flush=True)
    s = A.HipSession(hm, B, 200)
    nxt, lg = s.prefill(ids=ids, n_ids=n, want_logits=True)
    assert list(s.lengths()) == list(n)
    for b in range(B):
        st = O.State(c1g, 200)
        h = st.forward(O.embed(c1g, ids[b, : n[b]]))
        want = O.head(c1g, h[-1:])
        assert_logits_close(lg[b:b + 1], want, "row %d prefill" % b)
        assert nxt[b] == int(np.argmax(want[0]))
    out, _ = s.decode(nxt, 20)
    for b in range(B):
        want = c1g.generate(ids[b, : n[b]], 21, eos=-1)
        assert [int(nxt[b])] + list(out[:, b]) == list(want[n[b]:]), "row %d decode after prefill" % b


@pytest.mark.parametrize("nt", ["4,4,4", "3,3,3", "2,2,2"])
def test_prefill_tile_widths(c1g, nt, monkeypatch):
    """Every prefill GEMM tile width (128, 96 or 64 columns, forced for the
    QKV, residual and SwiGLU GEMMs) gives the oracle's logits at each row's
    last position.  The c1g GEMMs have 768, 256 and 1,366 columns, so some
    widths end in a partial tile; 400-odd rows use the prefill shape."""
    monkeypatch.setenv("DNN_HIP_PREFILL_NT", nt)
    hm = hip_model(c1g)
    rng = np.random.default_rng(77)
    B = 4
    n = rng.integers(60, 150, size=B).astype(np.int32)
    ids = rng.integers(0, 128, size=(B, int(n.max()))).astype(np.int32)
    s = A.HipSession(hm, B, 200)
    nxt, lg = s.prefill(ids=ids, n_ids=n, want_logits=True)
    for b in range(B):
        st = O.State(c1g, 200)
        h = st.forward(O.embed(c1g, ids[b, : n[b]]))
        want = O.head(c1g, h[-1:])
        assert_logits_close(lg[b:b + 1], want, "row %d prefill, tiles %s" % (b, nt))
        assert nxt[b] == int(np.argmax(want[0]))


@pytest.mark.parametrize("B,nmax", [(1, 1), (1, 32), (3, 20), (8, 8)])
def test_short_prefill_on_decode_gemms(c1g, B, nmax):
    """Prefills of at most 64 rows run the decode-shape GEMMs: the oracle's
    logits at each row's last position, then the oracle's generation."""
    hm = hip_model(c1g)
    rng = np.random.default_rng(300 + B * 7 + nmax)
    n = rng.integers(1, nmax + 1, size=B).astype(np.int32)
    assert int(n.sum()) <= 64
    ids = rng.integers(0, 128, size=(B, int(n.max()))).astype(np.int32)
    s = A.HipSession(hm, B, 80)
    nxt, lg = s.prefill(ids=ids, n_ids=n, want_logits=True)
    for b in range(B):
        st = O.State(c1g, 80)
        h = st.forward(O.embed(c1g, ids[b, : n[b]]))
        want = O.head(c1g, h[-1:])
        assert_logits_close(lg[b:b + 1], want, "row %d short prefill" % b)
        assert nxt[b] == int(np.argmax(want[0]))
    out, _ = s.decode(nxt, 12)
    for b in range(B):
        want = c1g.generate(ids[b, : n[b]], 13, eos=-1)
        assert [int(nxt[b])] + list(out[:, b]) == list(want[n[b]:]), "row %d decode after short prefill" % b


def test_prefill_c2_long_prompt(golden):
    """C2: a 288-token prompt prefilled at once (five 64-row tiles, 288-key
    causal attention) against the oracle's cached forward."""
    m = O.Model(8192, 768, 12, 12, 2048, 1088, seed=2)
    hm = hip_model(m)
    toks = np.array(golden["c2_tokens"][:288], dtype=np.int32)
    s = A.HipSession(hm, 1, 320)
    nxt, lg = s.prefill(ids=toks[None, :], want_logits=True)
    st = O.State(m, 288)
    h = st.forward(O.embed(m, toks))
    want = O.head(m, h[-1:])
    assert_logits_close(lg, want, "c2 prefill 288")
    assert nxt[0] == golden["c2_tokens"][288]


@pytest.mark.parametrize("B", [3, 16])
def test_prefill_prefix_lm(B):
    """Prefix-LM prefill (the VLM shape, vlm.c:497-517): embedding rows as a
    bidirectional prefix, then causal text tokens, ragged per row; against the
    oracle's prefix-LM cached forward (transformer.c:313-323), then greedy
    decode on from the prefill against the oracle continuing the same state."""
    V, D, L, H, F = 256, 128, 2, 2, 256
    m = O.Model(V, D, L, H, F, 128, seed=5, init="gpt2")
    hm = hip_model(m)
    rng = np.random.default_rng(300 + B)
    I = 70
    emb = rng.standard_normal((B, I, D)).astype(np.float32)
    n = rng.integers(1, 5, size=B).astype(np.int32)
    ids = rng.integers(0, V, size=(B, 4)).astype(np.int32)
    s = A.HipSession(hm, B, 128)
    nxt, lg = s.prefill(ids=ids, n_ids=n, embeds=emb, mode=1, prefix_len=I, want_logits=True)
    assert list(s.lengths()) == list(I + n)
    out, olg = s.decode(nxt, 6, want_logits=True)
    for b in range(B):
        st = O.State(m, 128)
        x = np.concatenate([emb[b], O.embed(m, ids[b, : n[b]])])
        h = st.forward(x, mode=1, prefix_len=I)
        want = O.head(m, h[-1:])
        assert_logits_close(lg[b:b + 1], want, "row %d prefix prefill" % b)
        tok = int(np.argmax(want[0]))
        assert nxt[b] == tok
        for t in range(6):
            h = st.forward(O.embed(m, np.array([tok], np.int32)))
            w = O.head(m, h)
            assert_logits_close(olg[t, b:b + 1], w, "row %d decode step %d" % (b, t))
            tok = int(np.argmax(w[0]))
            assert out[t, b] == tok, "row %d step %d" % (b, t)


@pytest.mark.parametrize("B", [1, 20])
def test_bf16_weights_match_rounded_oracle(B):
    """bf16 weight storage (W16A32, no reference counterpart): tokens and
    logits equal the oracle's fp32 arithmetic on the same bf16-rounded weights,
    to the same bar."""
    m = O.Model(128, 256, 4, 4, 683, 128, seed=11, init="gpt2")
    m.round_weights_bf16()
    hm = A.HipModel(m.V, m.D, m.L, m.H, m.F, m.params(), rope=m.rope_tables(), weights=A.WEIGHTS_BF16)
    rng = np.random.default_rng(400 + B)
    feed = rng.integers(0, 128, size=(6, B)).astype(np.int32)
    s = A.HipSession(hm, B, 64)
    ids, lg = s.decode(feed, 30, want_logits=True)
    assert s.kernel() == (3 if B <= 4 else 6)      # the persistent kernel's bf16 form, or the engine
    for b in range(B):
        want, wlg = m.generate(feed[:, b], 25, eos=-1, want_logits=True)
        assert list(ids[5:, b]) == list(want[6:]), "row %d" % b
        assert_logits_close(lg[5:, b], wlg, "row %d" % b)


@pytest.mark.parametrize("B,nmax", [(2, 20), (3, 60)])
def test_bf16_prefill_matches_rounded_oracle(B, nmax):
    """bf16 weights through the prefill (at most 64 rows: the decode-shape
    GEMMs; more: the prefill shape) and the decode after it: the oracle's
    fp32 arithmetic on the same bf16-rounded weights, to the same bar."""
    m = O.Model(128, 256, 4, 4, 683, 128, seed=13, init="gpt2")
    m.round_weights_bf16()
    hm = A.HipModel(m.V, m.D, m.L, m.H, m.F, m.params(), rope=m.rope_tables(), weights=A.WEIGHTS_BF16)
    rng = np.random.default_rng(500 + B + nmax)
    n = rng.integers(nmax // 2, nmax + 1, size=B).astype(np.int32)
    ids = rng.integers(0, 128, size=(B, int(n.max()))).astype(np.int32)
    s = A.HipSession(hm, B, 100)
    nxt, lg = s.prefill(ids=ids, n_ids=n, want_logits=True)
    for b in range(B):
        st = O.State(m, 100)
        h = st.forward(O.embed(m, ids[b, : n[b]]))
        want = O.head(m, h[-1:])
        assert_logits_close(lg[b:b + 1], want, "row %d bf16 prefill" % b)
        assert nxt[b] == int(np.argmax(want[0]))
    out, _ = s.decode(nxt, 10)
    for b in range(B):
        want = m.generate(ids[b, : n[b]], 11, eos=-1)
        assert [int(nxt[b])] + list(out[:, b]) == list(want[n[b]:]), "row %d bf16 decode after prefill" % b


def test_prefill_block_head_after_every_row_stopped():
    """An engine decode whose rows all stop at eos leaves the device step state
    marked done (the rest of its graph replays skip their work).  A prefill,
    a layer-level block and a head call on the same session afterwards must
    still compute: each equals the same call on a fresh session."""
    V, EOS = 512, 258
    m = O.Model(V, 256, 2, 4, 683, 64, seed=23)
    m.param_view(O.lib().orc_model_n_params(m.ptr) - 1)[EOS] = 50.0    # every step emits eos
    hm = hip_model(m)
    B = 8                                                               # the engine
    r = np.random.default_rng(5)
    feed = r.integers(0, V, size=(4, B)).astype(np.int32)
    feed[feed == EOS] = 1
    ids = r.integers(0, V, size=(B, 6)).astype(np.int32)
    x = r.standard_normal((B, 3, 256)).astype(np.float32)
    xh = r.standard_normal((5, 256)).astype(np.float32)

    s = A.HipSession(hm, B, 64)
    out, _ = s.decode(feed, 12, eos=EOS)
    assert s.kernel() == 6 and len(out) < 12 and (out[-1] == EOS).all()
    s.reset()
    nxt, lg = s.prefill(ids=ids, want_logits=True)
    y = s.block_forward(0, x, int(s.lengths()[0]))
    h = s.head_forward(xh)

    f = A.HipSession(hm, B, 64)
    nxt_f, lg_f = f.prefill(ids=ids, want_logits=True)
    y_f = f.block_forward(0, x, int(f.lengths()[0]))
    h_f = f.head_forward(xh)
    assert np.array_equal(nxt, nxt_f) and np.array_equal(lg, lg_f)
    assert np.array_equal(y, y_f)
    assert np.array_equal(h, h_f)
