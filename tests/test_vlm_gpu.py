"""vision_lm on the device (vlm.c:153-611) from a C caller of the reference's
API (tests/c/vlm_main.c), against fixtures the reference wrote
(tests/golden/gen_vlm.c): image embeddings of a 4D image (patch conv) and a
pre-patched 3D one (img_proj), the full prefix-LM forward, and greedy
vision_lm_generate with and without the KV cache.

Bars: ids identical; logits within max-abs 1e-3 / relative 1e-4 per row (the
north-star tolerance); image embeddings within 1e-5 (one fp32 dot product of
48 terms per value, summed in another order than the reference's)."""
import json
import os
import subprocess

import numpy as np
import pytest

from test_parity_gpu import assert_logits_close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DATA = os.path.join(ROOT, "tests", "golden", "data")


def test_vision_lm_generate_matches_reference(vlm_main, tmp_path):
    with open(os.path.join(DATA, "vlm_gen.json")) as f:
        g = json.load(f)
    print("vlm_main gen", flush=True)
    r = json.loads(subprocess.check_output([vlm_main, "gen", str(tmp_path)], text=True, timeout=300))
    assert r["params"] == g["vg_params"]

    def load(name, cols, d=str(tmp_path)):
        return np.fromfile(os.path.join(d, name), dtype=np.float32).reshape(-1, cols)

    for k in ("4", "3"):
        got, want = load("embeds%s.f32" % k, 128), load("vg_embeds%s.f32" % k, 128, DATA)
        np.testing.assert_allclose(got, want, atol=1e-5, rtol=0, err_msg="embeds" + k)
    assert_logits_close(load("forward4.f32", 96), load("vg_forward4.f32", 96, DATA), "vision_lm_forward")
    assert r["text_logits_shape"] == [1, 4, 96]
    assert r["tokens4_cache"] == g["vg_tokens4_cache"]
    assert r["tokens4_nocache"] == g["vg_tokens4_nocache"]
    assert r["tokens3_cache"] == g["vg_tokens3_cache"]
