"""The host library (dnn.c_amd/host) and the oracle built with
AddressSanitizer and UndefinedBehaviorSanitizer (gcc, CPU only; errors abort):
the paths that run without a GPU -- building the reference's weights through its
API, a DNNM checkpoint round trip, the tokenizer, vision_lm's parameters, the
oracle's cached and uncached C1 generation -- give the same results as the
plain builds and report nothing.  The device library is linked unchanged (not
instrumented) and never called."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "dnn.c_amd", "lib")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")


def host_sources():
    d = os.path.join(ROOT, "dnn.c_amd", "host")
    return sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(".c"))


@pytest.fixture(scope="module")
def san_build(built, tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not found")
    out = tmp_path_factory.mktemp("san")
    exes = {}
    for name in ("generate_main", "ckpt_main", "tok_main", "vlm_main"):
        exe = str(out / name)
        subprocess.check_call(["gcc", "-std=gnu11", *SAN, "-I" + os.path.join(ROOT, "include"),
                               "-I" + os.path.join(ROOT, "include", "dnn"),
                               os.path.join(ROOT, "tests", "c", name + ".c"), *host_sources(), "-o", exe,
                               "-L" + LIB, "-ldnn_hip", "-Wl,-rpath," + LIB, "-lm"])
        exes[name] = exe
    exe = str(out / "oracle_main")
    subprocess.check_call(["gcc", "-std=gnu11", *SAN, "-I" + os.path.join(ROOT, "oracle"),
                           os.path.join(ROOT, "tests", "c", "oracle_main.c"),
                           os.path.join(ROOT, "oracle", "dnn_oracle.c"), "-o", exe, "-lm"])
    exes["oracle_main"] = exe
    return exes


def run(exe, *args):
    p = subprocess.run([exe] + [str(a) for a in args], capture_output=True, text=True, timeout=600, env=ENV)
    assert p.returncode == 0 and "runtime error" not in p.stderr and "AddressSanitizer" not in p.stderr, p.stderr[-3000:]
    return p.stdout


def test_host_weights_under_sanitizers(san_build, golden):
    r = json.loads(run(san_build["generate_main"], 128, 256, 4, 4, 683, 256, 1, "synthetic", 101, 16, 0))
    assert r["params"] == golden["c1_params"]
    assert r["tokens"] == golden["c1_prompt"]
    r = json.loads(run(san_build["generate_main"], 128, 256, 4, 4, 683, 256, 11, "gpt2", 111, 16, 0))
    assert r["params"] == golden["c1g_params"]


def test_checkpoint_and_vlm_under_sanitizers(san_build, tmp_path):
    with open(os.path.join(ROOT, "tests", "golden", "data", "ckpt.json")) as f:
        g = json.load(f)
    ref = os.path.join(ROOT, "tests", "golden", "data", "ckpt_small.dnnm")
    r = json.loads(run(san_build["ckpt_main"], "load", ref, str(tmp_path / "again.dnnm")))
    assert r["loaded"] == g["ckpt_params"] and r["reloaded"] == g["ckpt_params"]
    with open(os.path.join(ROOT, "tests", "golden", "data", "vlm_gen.json")) as f:
        v = json.load(f)
    assert json.loads(run(san_build["vlm_main"], "params"))["params"] == v["vg_params"]


def test_tokenizer_under_sanitizers(san_build):
    with open(os.path.join(ROOT, "tests", "golden", "data", "tokenizer.json")) as f:
        want = json.load(f)
    assert json.loads(run(san_build["tok_main"])) == want


def test_oracle_under_sanitizers(san_build, golden):
    prompt = golden["c1_prompt"]
    r = json.loads(run(san_build["oracle_main"], 24, *prompt))
    assert r["tokens"] == golden["c1_tokens"][: len(prompt) + 24]
    assert r["nocache_agrees"] == 1
