"""GPU parity of the decode path against the oracle (itself bit-pinned to the
reference by test_oracle_golden.py) and the reference's fixtures.

Bars:
  * greedy token sequences identical to the reference's;
  * per-step logits within max-abs 1e-3 and relative 1e-4, the relative error
    being max|dlogit| / max|logit| over the step's vocabulary row.
"""
import json
import os
import subprocess

import numpy as np
import pytest

import dnn_amd as A
import oracle_lib as O
from golden_util import binf

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

ABS_TOL = 1e-3
REL_TOL = 1e-4


def assert_logits_close(got, want, what):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want).max(axis=-1)
    scale = np.abs(want).max(axis=-1)
    assert err.max() <= ABS_TOL, "%s: max |dlogit| %.3g" % (what, err.max())
    assert (err / scale).max() <= REL_TOL, "%s: max relative %.3g" % (what, (err / scale).max())


def hip_model(m):
    return A.HipModel(m.V, m.D, m.L, m.H, m.F, m.params(), rope=m.rope_tables())


@pytest.fixture(scope="module")
def c1():
    return O.Model(128, 256, 4, 4, 683, 256, seed=1)


@pytest.fixture(scope="module")
def c1g():
    return O.Model(128, 256, 4, 4, 683, 256, seed=11, init="gpt2")


@pytest.fixture(scope="module")
def c2():
    m = O.Model(8192, 768, 12, 12, 2048, 1088, seed=2)
    return m, hip_model(m)


@pytest.mark.parametrize("tag", ["c1", "c1g"])
def test_c1_greedy_tokens_and_logits(golden, c1, c1g, tag):
    m = c1 if tag == "c1" else c1g
    hm = hip_model(m)
    prompt = np.array(golden[tag + "_prompt"], dtype=np.int32)
    assert list(hm.generate(prompt, 240)) == golden[tag + "_tokens"]
    # teacher-forced on the reference's own ids: every step's logits
    s = A.HipSession(hm, 1, 256)
    toks = golden[tag + "_tokens"]
    _, lg = s.decode(np.array(toks[:-1]), len(toks) - 1, want_logits=True)
    assert_logits_close(lg[15:, 0], binf(tag + "_logits.f32", 128), tag)


def test_c2_tokens_match_reference(golden, c2):
    """The headline config: 32-token prompt, 512 greedy tokens, all identical."""
    _, hm = c2
    out = hm.generate(np.array(golden["c2_prompt"], dtype=np.int32), 512)
    assert list(out) == golden["c2_tokens"]


def test_c2_logits_first_steps(golden, c2):
    _, hm = c2
    s = A.HipSession(hm, 1, 64)
    toks = golden["c2_tokens"][:36]
    _, lg = s.decode(np.array(toks[:-1]), 35, want_logits=True)
    assert_logits_close(lg[31:, 0], binf("c2_logits4.f32", 8192), "c2 first 4 steps")


def test_c2_logits_late_steps_vs_oracle(golden, c2):
    """Teacher-forced positions 256..287 (KV history of up to 288 keys: five
    64-key attention chunks combined across workgroups)."""
    m, hm = c2
    toks = np.array(golden["c2_tokens"], dtype=np.int32)
    st = O.State(m, 288)
    h = st.forward(O.embed(m, toks[:288]))    # one cached pass over 288 rows
    want = O.head(m, h[-32:])
    s = A.HipSession(hm, 1, 288)
    _, lg = s.decode(toks[:288], 288, want_logits=True)
    assert_logits_close(lg[-32:, 0], want, "c2 positions 256-287")


def test_c2_gpt2_init_tokens(golden):
    m = O.Model(8192, 768, 12, 12, 2048, 1088, seed=12, init="gpt2")
    hm = hip_model(m)
    want = golden["c2g_tokens"]
    out = hm.generate(np.array(golden["c2g_prompt"], dtype=np.int32), len(want) - 32)
    assert list(out) == want


@pytest.mark.parametrize("B,kern", [(2, ""), (5, ""), (5, "3"), (8, ""), (8, "3"), (20, "")])
def test_batch_rows_match_independent_runs(c1g, monkeypatch, B, kern):
    """Each row of a batched decode equals its own B=1 run (rows differ in
    prompt length, so they switch from prompt to greedy at different steps);
    5 and 8 rows on the default (batched engine) and on the persistent kernel."""
    if kern:
        monkeypatch.setenv("DNN_HIP_DECODE_KERNEL", kern)
    hm = hip_model(c1g)
    rng = np.random.default_rng(B)
    lens = rng.integers(1, 9, size=B).astype(np.int32)
    feed = rng.integers(0, 128, size=(8, B)).astype(np.int32)
    steps = 40
    s = A.HipSession(hm, B, 64)
    ids, lg = s.decode(feed, steps, n_feed=lens, want_logits=True)
    for b in range(B):
        want, wlg = c1g.generate(feed[: lens[b], b], steps - lens[b] + 1, eos=-1, want_logits=True)
        got = list(feed[: lens[b], b]) + list(ids[lens[b] - 1:, b])
        assert got == list(want), "row %d" % b
        assert_logits_close(lg[lens[b] - 1:, b], wlg, "row %d" % b)
    assert list(s.lengths()) == [steps] * B
    assert s.kernel() == (3 if B <= 4 or kern == "3" else 6)


@pytest.mark.parametrize("B,splits", [(1, 2), (1, 3), (1, 4), (2, 4), (8, 4)])
def test_general_kernel_split_attention(monkeypatch, B, splits):
    """The general kernel with each head's keys split over several workgroups
    (DNN_HIP_ATT_SPLITS; the out_proj workgroups merge the partial softmax
    records): 600 positions, so every split walks several 32-key chunks and
    splits with no chunk occur at the first steps.  Every row's tokens and
    logits against the oracle."""
    steps = 600
    m = O.Model(128, 256, 4, 4, 683, steps + 8, seed=11, init="gpt2")
    hm = hip_model(m)
    rng = np.random.default_rng(steps + B)
    feed = rng.integers(0, 128, size=(4, B)).astype(np.int32)
    monkeypatch.setenv("DNN_HIP_DECODE_KERNEL", "3")
    monkeypatch.setenv("DNN_HIP_ATT_SPLITS", str(splits))
    s = A.HipSession(hm, B, steps + 8)
    ids, lg = s.decode(feed, steps, n_feed=np.full(B, 4, np.int32), want_logits=True)
    assert s.kernel() == 3 and s.att_splits() == splits
    for b in range(B):
        want, wlg = m.generate(feed[:, b], steps - 3, eos=-1, want_logits=True)
        assert list(ids[3:, b]) == list(want[4:]), "row %d" % b
        assert_logits_close(lg[3:, b], wlg, "row %d" % b)


def test_general_kernel_split_choice():
    """The automatic choice: one workgroup per head while each wavefront walks
    at most 4 chunks of 32 keys (histories up to 1024), then more; the tokens
    of the split launches against the oracle."""
    m = O.Model(128, 256, 4, 4, 683, 2200, seed=11, init="gpt2")
    hm = hip_model(m)
    s = A.HipSession(hm, 1, 2200)
    ids, _ = s.decode(np.array([5]), 1000)
    assert s.att_splits() == 1
    ids2, _ = s.decode(ids[-1:], 100)           # positions up to 1100: 35 chunks
    assert s.att_splits() == 2
    ids3, _ = s.decode(ids2[-1:], 1000)         # up to 2100: 66 chunks
    assert s.att_splits() == 3
    want = m.generate(np.array([5], dtype=np.int32), 2100, eos=-1)
    assert list(ids[:, 0]) + list(ids2[:, 0]) + list(ids3[:, 0]) == list(want[1:])


def test_eos_stops_generation():
    """A bias pushing id 258 to the top makes the first generated token EOS: the
    run stops there (gpt.c:339), on the device as in the oracle."""
    m = O.Model(300, 128, 2, 2, 256, 64, seed=3, init="gpt2")
    p = m.params()
    p[-1][258] = 50.0                      # lm_head.bias
    hm = A.HipModel(300, 128, 2, 2, 256, p, rope=m.rope_tables())
    prompt = O.prompt_ids(9, 300, 5)
    out = hm.generate(prompt, 20)
    assert list(out) == list(prompt) + [258]


def test_session_bounds_are_errors(c1g):
    hm = hip_model(c1g)
    s = A.HipSession(hm, 1, 8)
    with pytest.raises(A.HipError, match="max_seq"):
        s.decode(np.array([1]), 9)
    with pytest.raises(A.HipError, match="outside"):
        s.decode(np.array([128]), 1)
    ids, _ = s.decode(np.array([1]), 8)
    assert len(ids) == 8
    with pytest.raises(A.HipError, match="max_seq"):
        s.decode(ids[-1:], 1)
    s.reset()
    assert list(s.lengths()) == [0]


@pytest.mark.parametrize("grid", [4, 6, 9, 40])
def test_small_grids_match_default_grid(c1g, grid, monkeypatch):
    """The persistent kernel on grids down to one workgroup per role (a grid
    too small for the role planner's search is split by weight bytes, and
    every phase then runs many rounds): tokens and logits bit-identical to the
    default grid, since each output's summation order does not depend on how
    units map to workgroups (one key split, so the attention is the same)."""
    monkeypatch.setenv("DNN_HIP_ATT_SPLITS", "1")
    hm = hip_model(c1g)
    prompt = np.arange(1, 9, dtype=np.int32)
    ref = A.HipSession(hm, 1, 40)
    want, wlg = ref.decode(prompt, 24, want_logits=True)
    s = A.HipSession(hm, 1, 40)
    s.set_grid(grid)
    got, glg = s.decode(prompt, 24, want_logits=True)
    assert s.kernel() == 3 and s.grid() == grid and ref.grid() > 40
    assert np.array_equal(got, want) and np.array_equal(glg, wlg)


def test_small_grid_c2_shape(c2, monkeypatch):
    """The C2 shape (d=768) on 12 workgroups, below the searched splits (28):
    the same tokens and logits as the default grid."""
    monkeypatch.setenv("DNN_HIP_ATT_SPLITS", "1")
    _, hm = c2
    prompt = np.arange(3, 9, dtype=np.int32)
    ref = A.HipSession(hm, 1, 32)
    want, wlg = ref.decode(prompt, 10, want_logits=True)
    s = A.HipSession(hm, 1, 32)
    s.set_grid(12)
    got, glg = s.decode(prompt, 10, want_logits=True)
    assert s.grid() == 12
    assert np.array_equal(got, want) and np.array_equal(glg, wlg)


def test_large_batch_is_refused(c1g):
    """Sessions hold at most 64 rows; more is an error at creation."""
    hm = hip_model(c1g)
    with pytest.raises(A.HipError, match="outside"):
        A.HipSession(hm, 65, 16)


def test_multi_group_eos_keeps_rows_in_step(c1g):
    """More than 8 rows (the batched engine) with an EOS stop: rows that emit
    EOS early are run on greedily while others have not, so every row advances
    the same number of steps and each row's ids equal its own independent run.
    Rows 8..11 share one prompt and rows 0..7 another; the EOS id is one the
    second prompt emits early and the first never does."""
    hm = hip_model(c1g)
    B, steps = 12, 40
    rng = np.random.default_rng(7)
    pa, pb = rng.integers(0, 128, size=(2, 4)).astype(np.int32)
    ra = c1g.generate(pa, steps - 3, eos=-1)
    rb = c1g.generate(pb, steps - 3, eos=-1)
    cands = [j for j in range(4, 20) if ra[j] not in set(ra[4:j]) and ra[j] not in set(rb[4:])]
    if not cands:
        pytest.skip("no EOS id separates the two prompts for this seed")
    j = cands[0]
    eos = int(ra[j])
    feed = np.stack([pb] * 8 + [pa] * 4, axis=1)
    s = A.HipSession(hm, B, 64)
    ids, _ = s.decode(feed, steps, n_feed=np.full(B, 4, np.int32), eos=eos)
    assert ids.shape[0] == steps                # the first group never emits eos
    assert list(s.lengths()) == [steps] * B
    for b in range(B):
        ref = rb if b < 8 else ra
        assert list(ids[3:, b]) == list(ref[4:steps + 1]), "row %d" % b


@pytest.mark.parametrize("init,seed,pseed,key", [("synthetic", 1, 101, "c1"), ("gpt2", 11, 111, "c1g")])
def test_c_api_generate_matches_reference(generate_main, golden, init, seed, pseed, key):
    """A C caller of decoder_lm_generate (the reference's API) gets the
    reference's ids, weights built by the same API calls."""
    out = subprocess.check_output([generate_main, "128", "256", "4", "4", "683", "256", str(seed), init,
                                   str(pseed), "16", "240"], text=True, timeout=300)
    r = json.loads(out)
    assert r["params"] == golden[key + "_params"]
    assert r["tokens"] == golden[key + "_tokens"]


def test_c_api_nocache_and_sampling(generate_main, golden):
    nc = json.loads(subprocess.check_output([generate_main, "128", "256", "4", "4", "683", "256", "1",
                                             "synthetic", "101", "16", "24", "0", "0"], text=True, timeout=300))
    assert nc["tokens"] == golden["c1_nocache_tokens"]
    a = subprocess.check_output([generate_main, "128", "256", "4", "4", "683", "256", "11", "gpt2",
                                 "111", "16", "32", "0.8"], text=True, timeout=300)
    b = subprocess.check_output([generate_main, "128", "256", "4", "4", "683", "256", "11", "gpt2",
                                 "111", "16", "32", "0.8"], text=True, timeout=300)
    ra, rb = json.loads(a), json.loads(b)
    assert ra["tokens"] == rb["tokens"] and len(ra["tokens"]) == 48


SAMPLE_TIE = 5e-5


@pytest.mark.parametrize("case", ["c1g_t08", "c1g_t15", "c2g_t10"])
def test_c_api_sampling_matches_reference(generate_main, case):
    """decoder_lm_generate with temperature > 0 through the C API: the ids the
    reference itself drew for the same seed (tests/golden/gen_sample.c), the
    sampler and default RNG on the host (gpt.c:232-254, rng.c:33-36) fed with
    the device's logits.  Those logits differ from the reference's in the last
    bits (summation order), which moves every CDF edge by about that much: a
    draw can land in another token's interval only at a step where the uniform
    draw sat within SAMPLE_TIE of its interval's edge (the fixture records that
    distance per step).  Ids must match up to such a step, and the comparison
    ends there; a fixture whose every margin is larger must match entirely."""
    with open(os.path.join(ROOT, "tests", "golden", "data", "sample.json")) as f:
        ref = json.load(f)[case]
    out = subprocess.check_output([generate_main, str(ref["V"]), str(ref["D"]), str(ref["L"]), str(ref["H"]),
                                   str(ref["F"]), str(ref["P"] + ref["new"]), str(ref["seed"]), "gpt2",
                                   str(ref["prompt_seed"]), str(ref["P"]), str(ref["new"]), repr(ref["temp"])],
                                  text=True, timeout=300)
    got, want, P = json.loads(out)["tokens"], ref["tokens"], ref["P"]
    assert got[:P] == want[:P]
    for t, m in enumerate(ref["margins"]):
        if P + t >= len(want):
            break
        if got[P + t] != want[P + t]:
            assert m < SAMPLE_TIE, "%s: draw %d differs (%d vs %d) with margin %.3g" % (case, t, got[P + t], want[P + t], m)
            print("%s: draw %d differs at margin %.2e (a CDF edge): comparison ends there" % (case, t, m), flush=True)
            return
    assert got == want
    print("%s: %d sampled ids identical (smallest margin %.2e)" % (case, len(want) - P, min(ref["margins"])), flush=True)


def test_checkpoint_load_then_generate(ckpt_main):
    """Generate on a model's own weights (mirrored to HBM), module_load a
    checkpoint the reference wrote, generate again: the device mirror follows
    the new weights and the ids are the ones the reference generated from that
    checkpoint."""
    with open(os.path.join(ROOT, "tests", "golden", "data", "ckpt.json")) as f:
        g = json.load(f)
    ref = os.path.join(ROOT, "tests", "golden", "data", "ckpt_small.dnnm")
    r = json.loads(subprocess.check_output([ckpt_main, "gen", ref], text=True, timeout=120))
    assert r["loaded"] == g["ckpt_tokens"]
    assert r["own"][:5] == g["ckpt_tokens"][:5] and r["own"] != g["ckpt_tokens"]
