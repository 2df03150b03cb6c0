"""The C-ABI libraries load and export every symbol their headers declare.
No device calls: these run without a GPU."""
import ctypes as C
import os
import re
import subprocess

import pytest

import dnn_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    """Function names declared in a C header (top-level prototypes)."""
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if not n.startswith(("if", "for", "while", "return", "sizeof"))))


def exported(lib):
    out = subprocess.check_output(["nm", "-D", "--defined-only", lib], text=True)
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_dnn_hip_exports_every_declared_symbol(built):
    names = declared(os.path.join(ROOT, "include", "dnn_hip.h"))
    assert set(names) == set(dnn_amd.HIP_SYMBOLS)
    assert set(names) <= exported(dnn_amd.HIP_LIB)


def test_host_api_exports_every_declared_symbol(built):
    have = exported(dnn_amd.AMD_LIB)
    missing = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include", "dnn"))):
        for n in declared(os.path.join(ROOT, "include", "dnn", h)):
            if n not in have:
                missing.append((h, n))
    assert not missing, missing


def test_libraries_load_without_a_device(built):
    C.CDLL(dnn_amd.HIP_LIB)
    L = C.CDLL(dnn_amd.AMD_LIB)
    L.dnn_seed.argtypes = [C.c_uint64]
    L.dnn_seed(1)


def test_error_string_is_empty_initially(built):
    assert dnn_amd.hip().dnn_hip_last_error() == b""


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(dnn_amd, "_hip", None)
    monkeypatch.setattr(dnn_amd, "HIP_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(dnn_amd.HipError):
        dnn_amd.hip()
