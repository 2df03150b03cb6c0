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


# ---- the drop-in boundary: our declarations against the reference's own ----

REF_INCLUDE = "/root/reference/include"

# the functions the boundary covers: generation, layer forwards, ops, pools,
# context, KV cache, RoPE, vision_lm generation
BOUNDARY = [
    "decoder_lm_create", "decoder_lm_init_weights", "decoder_lm_enable_rope", "decoder_lm_generate",
    "decoder_lm_lm_head_forward", "decoder_lm_argmax_token", "decoder_lm_forward", "decoder_lm_forward_embeds",
    "decoder_lm_forward_embeds_ex", "decoder_lm_hidden_from_embeds", "decoder_lm_hidden_from_embeds_ex",
    "decoder_lm_token_embeds", "kv_cache_create", "kv_cache_append", "kv_cache_get_K", "kv_cache_get_V",
    "transformer_block_create", "transformer_block_forward", "transformer_block_forward_ex",
    "transformer_block_forward_cached", "transformer_block_forward_cached_ex", "linear_create", "linear_forward",
    "rms_norm_create", "rms_norm_forward", "swiglu_ffn_create", "swiglu_ffn_forward", "embedding_create",
    "embedding_forward", "tensor_matmul_add", "tensor_rms_norm", "tensor_rope", "tensor_rope_freqs_init",
    "tensor_split_qkv_heads", "tensor_split_heads", "tensor_merge_heads", "tensor_add", "tensor_swiglu",
    "tensor_embedding", "tensor_cat", "tensor_zeros", "tensor_zeros_data", "tensor_randn", "tensor_slice",
    "tensor_reshape", "tensor_flatten", "tensor_numel", "tensor_data_ptr", "mem_pool_create", "mem_pool_destroy",
    "mem_pool_reset", "mem_pool_mark", "mem_pool_release", "_mem_pool_alloc", "_mem_pool_alloc_nz", "dnn_ctx_init",
    "dnn_ctx_destroy", "dnn_seed", "dnn_rng_seed", "dnn_rng_uniform", "dnn_rng_normal", "dnn_rng_uniform_int",
    "dnn_no_grad_enter", "dnn_no_grad_exit", "dnn_grad_enabled", "module_parameters", "module_save",
    "module_load", "vision_lm_generate",
]
STRUCTS = ["tensor", "mem_pool", "dnn_ctx", "linear", "rms_norm", "embedding", "swiglu_ffn", "transformer_block",
           "kv_cache", "decoder_lm"]


def _clean(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)


def _headers(d):
    return "\n".join(_clean(open(os.path.join(d, h)).read()) for h in sorted(os.listdir(d)) if h.endswith(".h"))


def _param_type(p):
    """A parameter's type without its name: 'const tensor *x' -> 'const tensor*'."""
    p = " ".join(p.replace("*", " * ").split())
    p = re.sub(r"\[\s*\d*\s*\]$", " *", p).strip()
    toks = p.split()
    if len(toks) > 1 and re.match(r"^[A-Za-z_]\w*$", toks[-1]) and toks[-1] not in (
            "int", "float", "char", "void", "double", "size_t", "tensor", "unsigned"):
        toks = toks[:-1]
    return " ".join(toks).replace(" *", "*").replace("struct ", "")


def _prototypes(text):
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w \t\*]*?)\b([A-Za-z_]\w*)\s*\(([^;{}()]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ret = " ".join(ret.replace("*", " * ").split()).replace(" *", "*").replace("struct ", "")
        ps = [] if params.strip() in ("", "void") else [_param_type(p) for p in params.split(",")]
        out[name] = (ret, tuple(ps))
    return out


def _struct_fields(text, name):
    m = re.search(r"typedef\s+struct\s*\w*\s*\{([^{}]*)\}\s*" + name + r"\s*;", text, flags=re.S)
    if not m:
        m = re.search(r"struct\s+" + name + r"\s*\{([^{}]*)\}\s*;", text, flags=re.S)
    assert m, name
    fields = []
    for f in m.group(1).split(";"):
        f = " ".join(f.replace("*", " * ").split())
        if f:
            fields.append(re.sub(r"\s*:\s*", ":", f).replace(" * ", "*").replace("struct ", ""))
    return fields


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers absent (they exist in the dev container)")
def test_boundary_prototypes_match_reference():
    """Every boundary function is declared in include/dnn with the reference's
    return and parameter types (parameter names may differ), so a reference
    caller compiles unchanged."""
    ref = _prototypes(_headers(REF_INCLUDE))
    ours = _prototypes(_headers(os.path.join(ROOT, "include", "dnn")))
    bad = []
    for n in BOUNDARY:
        assert n in ref, "not a reference function: " + n
        if n not in ours:
            bad.append((n, "missing"))
        elif ours[n] != ref[n]:
            bad.append((n, ours[n], ref[n]))
    assert not bad, bad


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers absent (they exist in the dev container)")
def test_boundary_structs_match_reference():
    """The structs a caller allocates or reads have the reference's fields in
    the reference's order and types."""
    ref, ours = _headers(REF_INCLUDE), _headers(os.path.join(ROOT, "include", "dnn"))
    bad = [(s, _struct_fields(ours, s), _struct_fields(ref, s)) for s in STRUCTS
           if _struct_fields(ours, s) != _struct_fields(ref, s)]
    assert not bad, bad


def test_boundary_functions_exported(built):
    have = exported(dnn_amd.AMD_LIB)
    assert not [n for n in BOUNDARY if n not in have]
