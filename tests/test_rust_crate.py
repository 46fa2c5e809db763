"""The Rust FFI crate (rust/darkforest-hip) against the C headers, on the CPU.

Cargo and rustc are not installed in this build's container, so the crate cannot be compiled here.
This test parses both sides instead: every function declared in include/dfattn.h and
include/dfgpt2.h must appear in an `extern "C"` block of the crate's sources with the same name,
the same number of arguments and the same type for each argument and for the result (C types
mapped to their Rust FFI equivalents: `const float *` is `*const f32`, `size_t` is `usize`,
`hipStream_t` and `void *` are `*mut c_void`, ...); no extern function may be missing from a header.
Planted mistakes (an argument's type changed, one dropped, a result type changed, a declaration
removed) each make the comparison fail. The build script must build the library with the repo's
Makefile (hipcc, gfx950) and link libdfattn and the HIP runtime; the constants must equal the
header's.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "rust", "darkforest-hip")
HEADERS = [os.path.join(ROOT, "include", h) for h in ("dfattn.h", "dfgpt2.h")]

# C type (normalised) -> Rust FFI type. Written from the C ABI, not from the crate.
C_TO_RUST = {
    "void": None, "int": "c_int", "float": "f32", "size_t": "usize", "uint32_t": "u32", "int32_t": "i32",
    "const float *": "*const f32", "float *": "*mut f32",
    "const void *": "*const c_void", "void *": "*mut c_void", "hipStream_t": "*mut c_void",
    "const int32_t *": "*const i32", "const uint16_t *": "*const u16", "uint16_t *": "*mut u16",
    "const uint32_t *": "*const u32", "uint32_t *": "*mut u32", "const char *": "*const c_char",
    "dfattn_context *": "*mut DfattnContext", "const dfattn_context *": "*const DfattnContext",
    "dfattn_context **": "*mut *mut DfattnContext",
}


def _norm_c_type(t):
    t = " ".join(t.replace("*", " * ").split())
    return t.replace("* *", "**")


def c_declarations(text):
    """name -> (result type, [argument types]) of every function declared in a C header."""
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w \*]*?)\b(\w+)\s*\(([^;{()]*)\)\s*;", text):
        ret, name, args = _norm_c_type(m.group(1)), m.group(2), m.group(3).strip()
        types = []
        if args and args != "void":
            for a in args.split(","):
                a = _norm_c_type(a)
                base = re.sub(r"\s*\b\w+$", "", a)  # drop the parameter name
                types.append(base)
        out[name] = (ret, types)
    return out


def rust_declarations(text):
    """name -> (result type or None, [argument types]) of every fn inside `extern "C"` blocks."""
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for block in re.finditer(r'extern\s+"C"\s*\{(.*?)\n\}', text, flags=re.S):
        for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block.group(1), flags=re.S):
            name, args, ret = m.group(1), m.group(2), m.group(3)
            types = [" ".join(a.split(":", 1)[1].split()) for a in args.split(",") if a.strip()]
            out[name] = (" ".join(ret.split()) if ret else None, types)
    return out


def crate_sources():
    src = os.path.join(CRATE, "src")
    return "\n".join(open(os.path.join(src, f)).read() for f in sorted(os.listdir(src)) if f.endswith(".rs"))


def header_declarations():
    decls = {}
    for h in HEADERS:
        decls.update(c_declarations(open(h).read()))
    return decls


def mismatches(c_decls, r_decls):
    problems = []
    for name, (ret, args) in c_decls.items():
        if name not in r_decls:
            problems.append(f"{name}: not declared in the crate")
            continue
        r_ret, r_args = r_decls[name]
        want_ret = C_TO_RUST[ret]
        if want_ret != r_ret:
            problems.append(f"{name}: result {r_ret} against C {ret}")
        if len(args) != len(r_args):
            problems.append(f"{name}: {len(r_args)} arguments against C's {len(args)}")
            continue
        for i, (ca, ra) in enumerate(zip(args, r_args)):
            if C_TO_RUST[ca] != ra:
                problems.append(f"{name}: argument {i} is {ra} against C {ca}")
    for name in r_decls:
        if name not in c_decls:
            problems.append(f"{name}: declared in the crate but in no header")
    return problems


def test_every_header_function_is_declared_with_its_signature():
    c_decls, r_decls = header_declarations(), rust_declarations(crate_sources())
    assert len(c_decls) >= 70, len(c_decls)
    assert mismatches(c_decls, r_decls) == []


@pytest.mark.parametrize("plant, expect", [
    (lambda s: s.replace("pub fn dfattn_bwd_main(q: *const f32", "pub fn dfattn_bwd_main(q: *mut f32", 1),
     "dfattn_bwd_main: argument 0"),
    (lambda s: s.replace("scale: f32, causal: u32, grad_row_stride: u32", "scale: f32, causal: u32", 1),
     "dfattn_bwd_main_strided: 12 arguments"),
    (lambda s: s.replace("pub fn dfattn_bwd_workspace_bytes(n_heads: u32, seq_len: u32, d_head: u32) -> usize",
                         "pub fn dfattn_bwd_workspace_bytes(n_heads: u32, seq_len: u32, d_head: u32) -> u32", 1),
     "dfattn_bwd_workspace_bytes: result u32"),
    (lambda s: re.sub(r"\n\s*pub fn darkforest_sync\(\);", "", s, count=1), "darkforest_sync: not declared"),
    (lambda s: s.replace("n_rows: u32,\n                                    dim: u32, rows_in_table: u32, stream: *mut c_void",
                         "n_rows: usize,\n                                    dim: u32, rows_in_table: u32, stream: *mut c_void", 1),
     "dfgpt2_embedding_forward: argument 3"),
])
def test_planted_signature_changes_are_caught(plant, expect):
    src = crate_sources()
    planted = plant(src)
    assert planted != src, "the planted change did not apply"
    problems = mismatches(header_declarations(), rust_declarations(planted))
    assert any(expect in p for p in problems), problems


def test_constants_match_the_header():
    header = open(HEADERS[0]).read()
    ffi = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    for name, value in re.findall(r"\b(DFATTN_\w+)\s*=\s*(-?\d+)", header):
        assert re.search(rf"pub const {name}: c_int = {value};", ffi), name
    for name, value in re.findall(r"#define (DFATTN_(?:BWD|KV)_\w+) (\d+)u", header):
        assert re.search(rf"pub const {name}: u32 = {value};", ffi), name
    assert "#define DFATTN_NOALLOC_SCRATCH_BYTES (32u << 20)" in header
    assert "pub const DFATTN_NOALLOC_SCRATCH_BYTES: usize = 32 << 20;" in ffi


def test_build_script_and_manifest():
    build = open(os.path.join(CRATE, "build.rs")).read()
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'Command::new("make")' in build and '.join("csrc")' in build
    assert "cargo:rustc-link-lib=dylib=dfattn" in build and "cargo:rustc-link-lib=dylib=amdhip64" in build
    make = open(os.path.join(ROOT, "dark-forest_amd", "csrc", "Makefile")).read()
    assert "ARCH     ?= gfx950" in make and "--offload-arch=$(ARCH)" in make
    assert 'name = "darkforest-hip"' in cargo and 'build = "build.rs"' in cargo and 'links = "dfattn"' in cargo
