"""Host side of the drop-in C API (include/dnn, libdnn_amd.so), no device:
a caller written against the reference's API builds the same weights and prompt
the reference built from the same seeds, and the DNNM state dict round-trips."""
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(exe, *args):
    out = subprocess.check_output([exe] + [str(a) for a in args], text=True, timeout=300)
    return json.loads(out)


@pytest.mark.parametrize("init,seed,pseed,key", [
    ("synthetic", 1, 101, "c1"),
    ("gpt2", 11, 111, "c1g"),
])
def test_c_api_builds_reference_weights_c1(generate_main, golden, init, seed, pseed, key):
    r = run(generate_main, 128, 256, 4, 4, 683, 256, seed, init, pseed, 16, 0)
    assert r["params"] == golden[key + "_params"]
    assert r["tokens"] == golden[key + "_prompt"]


def test_c_api_builds_reference_weights_c2(generate_main, golden):
    r = run(generate_main, 8192, 768, 12, 12, 2048, 1088, 2, "synthetic", 102, 32, 0)
    assert r["params"] == golden["c2_params"]
    assert r["tokens"] == golden["c2_prompt"]


def test_c_api_create_only_weights(generate_main, golden):
    r = run(generate_main, 128, 256, 4, 4, 683, 256, 7, "create", 1, 4, 0)
    assert r["params"] == golden["c1_create_params"]


def test_vision_lm_weights_match_reference(vlm_main):
    """vision_lm_create + vision_lm_init_weights + enable_rope through the
    reference's API give the reference's parameters bit for bit (patch conv,
    img_proj, the decoder, image positions; vlm.c:20-127)."""
    with open(os.path.join(ROOT, "tests", "golden", "data", "vlm_gen.json")) as f:
        g = json.load(f)
    r = json.loads(subprocess.check_output([vlm_main, "params"], text=True, timeout=120))
    assert r["params"] == g["vg_params"]
    assert r["n_params"] == 357600


def test_dnnm_checkpoint_round_trip(ckpt_main, tmp_path):
    """A DNNM checkpoint the reference's module_save wrote (module.c:208-230)
    loads strictly into a model of other weights and gives the reference's
    parameters bit for bit; module_save here writes the same bytes back, and
    that file loads into a third model."""
    with open(os.path.join(ROOT, "tests", "golden", "data", "ckpt.json")) as f:
        g = json.load(f)
    ref = os.path.join(ROOT, "tests", "golden", "data", "ckpt_small.dnnm")
    out = str(tmp_path / "again.dnnm")
    r = json.loads(subprocess.check_output([ckpt_main, "load", ref, out], text=True, timeout=120))
    assert r["before"] != g["ckpt_params"]
    assert r["loaded"] == g["ckpt_params"]
    assert r["reloaded"] == g["ckpt_params"]
    with open(ref, "rb") as a, open(out, "rb") as b:
        assert a.read() == b.read()


def test_tokenizer_matches_reference(built, tmp_path):
    """tests/c/tok_main.c (the reference's tokenizer API only) built against
    include/dnn prints what the same file printed built against the reference:
    byte ids with BOS/EOS, the chat template's special strings (and a
    truncated one left as bytes), decode dropping BOS/EOS/PAD and mapping
    other ids to '?', the tensor round trip, empty input."""
    exe = str(tmp_path / "tok_main")
    libdir = os.path.join(ROOT, "dnn.c_amd", "lib")
    subprocess.check_call(["gcc", "-std=gnu11", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include", "dnn"),
                           os.path.join(ROOT, "tests", "c", "tok_main.c"), "-o", exe,
                           "-L" + libdir, "-ldnn_amd", "-Wl,-rpath," + libdir, "-lm"])
    got = subprocess.check_output([exe], text=True, timeout=60)
    with open(os.path.join(ROOT, "tests", "golden", "data", "tokenizer.json")) as f:
        want = f.read()
    assert json.loads(got) == json.loads(want)
