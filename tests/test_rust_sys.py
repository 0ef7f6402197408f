"""The Rust binding crates under rust/ are text in this image (no cargo or
rustc), so these tests hold them to the C header instead of a compiler:

- rust/swiftllm-hip-sys/src/lib.rs declares every function of
  include/swiftllm_hip.h and nothing else, with the same parameter names in
  the same order and the Rust type of each C type; its repr(C) structs have
  the header structs' fields, and its status constants the header's values.
- rust/swiftllm-hip/src/bindings.rs keeps the signatures of the reference's
  safe bindings (crates/swiftllm-cuda/src/bindings.rs) for the functions on
  this path, so a crate calling those compiles against it unchanged.
"""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "swiftllm_hip.h"
SYS = ROOT / "rust" / "swiftllm-hip-sys" / "src" / "lib.rs"
SAFE = ROOT / "rust" / "swiftllm-hip" / "src" / "bindings.rs"

# C type (whitespace-normalised, '*' attached) -> Rust type in the -sys crate.
C_TO_RUST = {
    "void*": "*mut c_void",
    "const void*": "*const c_void",
    "void* const*": "*const *mut c_void",
    "int": "c_int",
    "int*": "*mut c_int",
    "const int*": "*const c_int",
    "int32_t*": "*mut i32",
    "const int32_t*": "*const i32",
    "int64_t*": "*mut i64",
    "const int64_t*": "*const i64",
    "const uint64_t*": "*const u64",
    "float": "c_float",
    "float*": "*mut c_float",
    "const float*": "*const c_float",
    "size_t": "usize",
    "long long": "c_longlong",
    "hipStream_t": "hipStream_t",
    "const char*": "*const c_char",
    "const swiftllm_paged_attention_params*": "*const swiftllm_paged_attention_params",
    "const swiftllm_reshape_cache_params*": "*const swiftllm_reshape_cache_params",
}


def _norm_c(t):
    t = " ".join(t.replace("*", " * ").split())
    return t.replace(" *", "*")


def c_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
    text = re.sub(r"typedef\s+(enum|struct)\s+\w+\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b([a-z_]\w*)\s*\(([^;{}]*?)\)\s*;", text, flags=re.S):
        ret, name, params = _norm_c(m.group(1)), m.group(2), " ".join(m.group(3).split())
        plist = []
        if params != "void":
            for p in params.split(","):
                p = _norm_c(p)
                ty, pname = p.rsplit(" ", 1) if not p.endswith("*") else (p, "")
                if pname.startswith("*"):
                    ty, pname = ty + "*", pname.lstrip("*")
                plist.append((_norm_c(ty), pname))
        out[name] = (ret, plist)
    return out


def _strip_rust_comments(text):
    return re.sub(r"//[^\n]*", "", text)


def rust_extern_functions():
    text = _strip_rust_comments(SYS.read_text())
    block = re.search(r'extern\s+"C"\s*\{(.*)\n\}', text, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, flags=re.S):
        name, params, ret = m.group(1), " ".join(m.group(2).split()), m.group(3)
        plist = []
        for p in [p.strip() for p in params.split(",") if p.strip()]:
            pname, ty = [x.strip() for x in p.split(":", 1)]
            plist.append((" ".join(ty.split()), pname))
        out[name] = (" ".join(ret.split()) if ret else None, plist)
    return out


def test_sys_crate_declares_exactly_the_header_functions():
    c, r = c_functions(), rust_extern_functions()
    assert len(c) >= 30
    assert sorted(c) == sorted(r)


@pytest.mark.parametrize("name", sorted(c_functions()))
def test_sys_crate_signature_matches_header(name):
    cret, cparams = c_functions()[name]
    rret, rparams = rust_extern_functions()[name]
    assert (None if cret == "void" else C_TO_RUST[cret]) == rret, f"{name}: return type"
    assert [p for _, p in cparams] == [p for _, p in rparams], f"{name}: parameter names"
    assert [C_TO_RUST[t] for t, _ in cparams] == [t for t, _ in rparams], f"{name}: parameter types"


def _c_structs():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        fields = [_norm_c(f).rsplit(" ", 1) for f in m.group(2).split(";") if f.strip()]
        out[m.group(3)] = [(C_TO_RUST[t], n) for t, n in fields]
    return out


def _rust_structs():
    text = _strip_rust_comments(SYS.read_text())
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\][^{]*?pub\s+struct\s+(\w+)\s*\{(.*?)\}", text, flags=re.S):
        fields = []
        for f in [f.strip() for f in m.group(2).split(",") if f.strip()]:
            n, t = [x.strip() for x in f.replace("pub ", "").split(":", 1)]
            fields.append((t, n))
        out[m.group(1)] = fields
    return out


def test_sys_crate_structs_match_header():
    c, r = _c_structs(), _rust_structs()
    assert sorted(c) == sorted(r) == ["swiftllm_paged_attention_params",
                                      "swiftllm_reshape_cache_params"]
    for name in c:
        assert c[name] == r[name], name


def test_sys_crate_status_codes_match_header():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    enum = re.search(r"typedef\s+enum\s+swiftllm_status\s*\{(.*?)\}", text, flags=re.S).group(1)
    c = {n: int(v) for n, v in re.findall(r"(SWIFTLLM_\w+)\s*=\s*(-?\d+)", enum)}
    r = {n: int(v) for n, v in re.findall(r"pub const (SWIFTLLM_\w+): c_int = (-?\d+);", SYS.read_text())}
    assert c == r and len(c) == 7


# The reference's safe signatures for this path (crates/swiftllm-cuda/src/
# bindings.rs): name -> [(parameter, type)], all returning Result<()>.
REFERENCE_SAFE = {
    # bindings.rs:33-41
    "paged_attention_prefill": [("output", "*mut half::f16"), ("query", "*const half::f16"),
                                ("key_cache", "*const half::f16"), ("value_cache", "*const half::f16"),
                                ("slot_mapping", "*const i32"), ("context_lens", "*const i32"),
                                ("params", "&PagedAttentionParams")],
    # bindings.rs:57-65
    "paged_attention_decode": [("output", "*mut half::f16"), ("query", "*const half::f16"),
                               ("key_cache", "*const half::f16"), ("value_cache", "*const half::f16"),
                               ("block_tables", "*const i32"), ("context_lens", "*const i32"),
                               ("params", "&PagedAttentionParams")],
    # bindings.rs:95-102
    "reshape_and_cache": [("key", "*const half::f16"), ("value", "*const half::f16"),
                          ("key_cache", "*mut half::f16"), ("value_cache", "*mut half::f16"),
                          ("slot_mapping", "*const i32"), ("params", "&ReshapeCacheParams")],
    # bindings.rs:201-210
    "copy_blocks": [("key_caches", "&[*mut half::f16]"), ("value_caches", "&[*mut half::f16]"),
                    ("block_mapping", "*const i64"), ("num_pairs", "usize"), ("num_layers", "usize"),
                    ("num_kv_heads", "usize"), ("head_dim", "usize"), ("block_size", "usize")],
    # bindings.rs:226-232
    "swap_blocks": [("src", "*const half::f16"), ("dst", "*mut half::f16"),
                    ("block_mapping", "*const i64"), ("num_pairs", "usize"),
                    ("block_size_bytes", "usize")],
}

# bindings.rs:8-30 and :78-92: field lists of the params structs.
REFERENCE_PARAMS = {
    "PagedAttentionParams": [("num_seqs", "usize"), ("num_heads", "usize"), ("num_kv_heads", "usize"),
                             ("head_dim", "usize"), ("block_size", "usize"), ("scale", "f32"),
                             ("max_context_len", "usize")],
    "ReshapeCacheParams": [("num_tokens", "usize"), ("num_kv_heads", "usize"), ("head_dim", "usize"),
                           ("block_size", "usize")],
}


def _safe_functions():
    text = _strip_rust_comments(SAFE.read_text())
    out = {}
    for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\((.*?)\)\s*->\s*([^{]+?)\s*\{", text, flags=re.S):
        plist = []
        for p in [p.strip() for p in " ".join(m.group(2).split()).split(",") if p.strip()]:
            n, t = [x.strip() for x in p.split(":", 1)]
            plist.append((n, t))
        out[m.group(1)] = (plist, m.group(3).strip())
    return out


def test_safe_bindings_keep_the_reference_signatures():
    got = _safe_functions()
    for name, params in REFERENCE_SAFE.items():
        assert name in got, name
        assert got[name][0] == params, name
        assert got[name][1] == "Result<()>", name


def test_safe_bindings_keep_the_reference_params_structs():
    text = _strip_rust_comments(SAFE.read_text())
    for name, fields in REFERENCE_PARAMS.items():
        body = re.search(r"pub\s+struct\s+" + name + r"\s*\{(.*?)\}", text, flags=re.S).group(1)
        got = [tuple(x.strip() for x in f.replace("pub ", "").split(":", 1))
               for f in body.split(",") if f.strip()]
        assert got == fields, name


def test_safe_bindings_call_only_declared_functions():
    declared = set(rust_extern_functions())
    called = set(re.findall(r"sys::(swiftllm_hip_\w+|launch_\w+)\s*\(", SAFE.read_text()))
    assert called and called <= declared, called - declared
