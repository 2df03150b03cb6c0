"""Greedy argmax on exact ties: the first index of the maximum (gpt.c:220-230,
a strict '>' scan from index 0).

The lm_head rows of TIED are all zero and share one large bias, so their
logits equal that bias exactly whatever the summation order, and they exceed
every other logit: every step is an exact tie among TIED, and the reference
picks min(TIED).  The ties span one 2-row unit of the batch-1 kernel's
lm_head (36, 37), one 16-column tile of the batched engine (36..38) and
separate workgroups of both (1000, 2047, 4095), so every level of each
reduction (within a wavefront, across wavefronts, across workgroups) meets a
tie.  The oracle is checked to see the same exact tie; the device must emit
the first index at every step of every row, on the persistent kernel (1-4
rows), the batched engine (8 and 32 rows) and the engine's prefill head.
"""
import numpy as np
import pytest

import dnn_amd as A
import oracle_lib as O
from test_parity_gpu import hip_model

pytestmark = pytest.mark.gpu

TIED = [36, 37, 38, 1000, 2047, 4095]
BIAS = 50.0
V, D, L, H, F = 4096, 256, 2, 4, 683
P, STEPS = 8, 12


@pytest.fixture(scope="module")
def tied():
    m = O.Model(V, D, L, H, F, 64, seed=21)
    emb = m.param_view(0).reshape(V, D)
    emb[TIED] = 0.0
    m.param_view(O.lib().orc_model_n_params(m.ptr) - 1)[TIED] = BIAS
    return m, hip_model(m)


def prompts(B):
    r = np.random.default_rng(77)
    ids = r.integers(0, V, size=(B, P)).astype(np.int32)
    ids[ids == TIED[0]] = 1          # prompts avoid the tied token itself
    return ids


def test_oracle_sees_exact_ties(tied):
    m, _ = tied
    out, lg = m.generate(prompts(1)[0], STEPS, eos=-1, want_logits=True)
    assert (out[P:] == TIED[0]).all()
    assert (lg[:, TIED] == BIAS).all()
    assert (np.delete(lg, TIED, axis=1) < BIAS).all()


@pytest.mark.parametrize("B", [1, 2, 4, 8, 32])
def test_device_argmax_takes_first_of_tied_maxima(tied, B):
    _, hm = tied
    ids = prompts(B)
    s = A.HipSession(hm, B, P + STEPS + 4)
    out, lg = s.decode(ids.T.copy(), P - 1 + STEPS, want_logits=True)
    assert s.kernel() == (3 if B <= 4 else 6)
    got = out[P - 1:]
    assert (lg[P - 1:][..., TIED] == BIAS).all(), "the tied logits are not exactly equal on the device"
    bad = np.argwhere(got != TIED[0])
    assert len(bad) == 0, "step %d row %d: token %d, want %d" % (bad[0][0], bad[0][1], got[tuple(bad[0])], TIED[0])


def test_engine_prefill_head_takes_first_of_tied_maxima(tied):
    _, hm = tied
    B = 16
    ids = prompts(B)
    lens = np.array([3 + (b % 6) for b in range(B)], dtype=np.int32)
    s = A.HipSession(hm, B, P + STEPS + 4)
    nxt, lg = s.prefill(ids=ids, n_ids=lens, want_logits=True)
    assert (lg[:, TIED] == BIAS).all()
    assert (np.asarray(nxt) == TIED[0]).all(), nxt
    out, _ = s.decode(nxt, STEPS)
    assert (out == TIED[0]).all()
