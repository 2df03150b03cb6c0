import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "dnn.c_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _make(*args):
    subprocess.check_call(["make", "-s"] + list(args))


@pytest.fixture(scope="session")
def built():
    """Builds the product and the oracle if their libraries are missing."""
    lib = os.path.join(ROOT, "dnn.c_amd", "lib", "libdnn_amd.so")
    if not os.path.exists(lib):
        _make("-C", os.path.join(ROOT, "dnn.c_amd"))
    if not os.path.exists(os.path.join(ROOT, "oracle", "_build", "liboracle.so")):
        _make("-C", os.path.join(ROOT, "oracle"))
    return ROOT


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "data", "index.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def generate_main(built, tmp_path_factory):
    """tests/c/generate_main.c built against include/dnn + libdnn_amd.so."""
    exe = str(tmp_path_factory.mktemp("c") / "generate_main")
    libdir = os.path.join(ROOT, "dnn.c_amd", "lib")
    subprocess.check_call(["gcc", "-std=gnu11", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "c", "generate_main.c"), "-o", exe,
                           "-L" + libdir, "-ldnn_amd", "-Wl,-rpath," + libdir, "-lm"])
    return exe


@pytest.fixture(scope="session")
def vlm_main(built, tmp_path_factory):
    """tests/c/vlm_main.c (a vision_lm caller) built against include/dnn + libdnn_amd.so."""
    exe = str(tmp_path_factory.mktemp("c") / "vlm_main")
    libdir = os.path.join(ROOT, "dnn.c_amd", "lib")
    subprocess.check_call(["gcc", "-std=gnu11", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "c", "vlm_main.c"), "-o", exe,
                           "-L" + libdir, "-ldnn_amd", "-Wl,-rpath," + libdir, "-lm"])
    return exe


@pytest.fixture(scope="session")
def ckpt_main(built, tmp_path_factory):
    """tests/c/ckpt_main.c (module_save / module_load caller) built against libdnn_amd.so."""
    exe = str(tmp_path_factory.mktemp("c") / "ckpt_main")
    libdir = os.path.join(ROOT, "dnn.c_amd", "lib")
    subprocess.check_call(["gcc", "-std=gnu11", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "c", "ckpt_main.c"), "-o", exe,
                           "-L" + libdir, "-ldnn_amd", "-Wl,-rpath," + libdir, "-lm"])
    return exe
