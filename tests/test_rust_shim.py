"""The Rust bindings (unillm_amd/rust) against the C header they bind.

No Rust toolchain exists in this build environment, so the crate is checked as
text: its extern "C" block declares exactly the header's functions, with the
same parameter names, the Rust type of every C type and the same return types;
its constants equal the header's #defines; build.rs compiles the same sources
with the same device flags as unillm_amd/build.py; Cargo.toml has no
dependencies.
"""
import os
import re

from unillm_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "unillm_hip.h")
CRATE = os.path.join(ROOT, "unillm_amd", "rust")

C_TO_RUST = {
    "int": "c_int", "int64_t": "i64", "size_t": "usize", "float": "f32",
    "const char*": "*const c_char",
    "const void*": "*const c_void", "void*": "*mut c_void", "void**": "*mut *mut c_void",
    "const float*": "*const f32", "float*": "*mut f32",
    "int*": "*mut c_int", "int64_t*": "*mut i64", "size_t*": "*mut usize",
    "const unillm_qweight*": "*const unillm_qweight", "unillm_qweight*": "*mut unillm_qweight",
    "unillm_qweight**": "*mut *mut unillm_qweight",
    "const unillm_kv_cache*": "*const unillm_kv_cache",
    "unillm_kv_cache*": "*mut unillm_kv_cache", "unillm_kv_cache**": "*mut *mut unillm_kv_cache",
    "const unillm_graph*": "*const unillm_graph", "unillm_graph*": "*mut unillm_graph",
    "unillm_graph**": "*mut *mut unillm_graph",
}


def _strip_c_comments(s):
    return re.sub(r"/\*.*?\*/", " ", s, flags=re.S)


def header_functions():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(
            r"^\s*((?:const\s+)?\w+\s*\*?)\s*(unillm_hip_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        args = []
        params = " ".join(params.split())
        if params not in ("", "void"):
            for p in params.split(","):
                m = re.match(r"^(.*?)(\w+)$", p.strip())
                ctype = re.sub(r"\s*\*", "*", m.group(1).strip())
                args.append((m.group(2), C_TO_RUST[ctype]))
        ret = re.sub(r"\s*\*", "*", ret.strip())
        out[name] = (args, C_TO_RUST[ret])
    return out


def rust_functions():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = re.search(r'extern "C" \{(.*?)\n    \}', text, flags=re.S).group(1)
    out = {}
    for name, params, ret in re.findall(
            r"pub fn (unillm_hip_\w+)\(([^)]*)\)\s*->\s*([^;]+);", block, flags=re.S):
        args = []
        params = " ".join(params.split())
        if params:
            for p in params.split(","):
                if not p.strip():
                    continue
                n, t = (s.strip() for s in p.split(":", 1))
                args.append((n, t))
        out[name] = (args, " ".join(ret.split()))
    return out


def test_rust_extern_block_equals_header():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 29
    assert sorted(h) == sorted(r), (set(h) ^ set(r))
    for name in h:
        assert r[name] == h[name], (name, r[name], h[name])


def test_rust_constants_equal_header_defines():
    text = _strip_c_comments(open(HEADER).read())
    defines = {n: int(v) for n, v in
               re.findall(r"#define (UNILLM_(?:QTYPE|OK|ERR|PATH)\w*)\s+\(?(-?\d+)\)?", text)}
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    consts = {n: int(v) for n, v in re.findall(r"pub const (UNILLM_\w+): c_int = (-?\d+);", lib)}
    assert defines and consts == defines


def test_build_rs_matches_build_py():
    text = open(os.path.join(CRATE, "build.rs")).read()
    sources = re.findall(r'"(\w+\.hip)"', re.search(r"const SOURCES.*?\];", text, re.S).group(0))
    assert sources == build.SOURCES
    flags = re.findall(r'"([^"]+)"', re.search(r"const FLAGS.*?\];", text, re.S).group(0))
    assert flags == build.FLAGS
    libs = re.findall(r'"([^"]+)"', re.search(r"const LIBS.*?\];", text, re.S).group(0))
    assert libs == build.LIBS
    assert "--offload-arch=gfx950" in flags and "-packed-fp32-ops" in flags
    assert '"-shared"' in text


def test_cargo_toml_has_no_dependencies():
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    deps = toml.split("[dependencies]", 1)[1]
    assert not [ln for ln in deps.splitlines() if ln.strip() and not ln.startswith("#")]
    assert 'build = "build.rs"' in toml
