"""The Rust binding crate (rust/scratchtape-hip-sys) against the C header, on the CPU.

There is no Rust toolchain in this image, so the crate is checked by parsing: its #[repr(C)] structs
match the header's typedefs field for field (order, names, types, hence size), its extern "C" block
declares exactly the header's functions with the same parameter names and types and return type,
its constants carry the header's values, and its safe wrappers call only declared functions.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "scratchtape_hip.h")
CRATE = os.path.join(ROOT, "rust", "scratchtape-hip-sys")

C_SCALARS = {"int32_t": "i32", "int64_t": "i64", "uint64_t": "u64", "uint32_t": "u32", "uint8_t": "u8", "int8_t": "i8",
             "float": "f32", "double": "f64", "void": "c_void", "char": "c_char",
             "st_status": "st_status", "st_stream": "st_stream", "st_matref": "st_matref",
             "st_epilogue": "st_epilogue", "st_gemm": "st_gemm"}
SIZES = {"i32": 4, "i64": 8, "u64": 8, "u32": 4, "f32": 4, "f64": 8, "st_status": 4, "st_stream": 8}


def strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def strip_rust_comments(text):
    return re.sub(r"//[^\n]*", "", text)


def c_type_to_rust(ctype):
    """'const float *' -> '*const f32', 'int64_t' -> 'i64', 'st_stream' -> 'st_stream'."""
    t = " ".join(ctype.replace("*", " * ").split())
    stars = t.count("*")
    words = [w for w in t.split() if w != "*"]
    const = "const" in words
    base = [w for w in words if w != "const"]
    assert len(base) == 1, ctype
    rust = C_SCALARS[base[0]]
    assert stars <= 1, ctype
    if stars:
        rust = ("*const " if const else "*mut ") + rust
    return rust


def split_decl(decl):
    """'const float *x' -> ('const float *', 'x')."""
    decl = " ".join(decl.replace("*", " * ").split())
    m = re.match(r"^(.*?)\s*\b([A-Za-z_][A-Za-z0-9_]*)$", decl)
    assert m, decl
    return m.group(1).strip(), m.group(2)


def header_structs():
    text = strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        assert m.group(1) == m.group(3)
        fields = []
        for line in m.group(2).split(";"):
            line = " ".join(line.split())
            if not line:
                continue
            first, *rest = line.split(",")
            ctype, name = split_decl(first)
            fields.append((name, c_type_to_rust(ctype)))
            for extra in rest:  # `st_matref a, b, out;` / `int64_t batch, m, k, n;`
                fields.append((extra.strip(), c_type_to_rust(ctype)))
        out[m.group(1)] = fields
    return out


def header_functions():
    text = strip_c_comments(open(HEADER).read())
    text = re.sub(r"#[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\s*\b(st_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret = c_type_to_rust(m.group(1))
        params = []
        args = " ".join(m.group(3).split())
        if args and args != "void":
            for a in args.split(","):
                ctype, name = split_decl(a)
                params.append((name, c_type_to_rust(ctype)))
        out[m.group(2)] = (params, ret)
    return out


def header_defines():
    text = open(HEADER).read()
    return dict(re.findall(r"#define\s+(ST_[A-Z_]+)\s+(\S.*?)\s*(?:/\*.*)?$", text, flags=re.M))


def rust_source(name):
    return open(os.path.join(CRATE, "src", name)).read()


def rust_structs(text=None):
    text = strip_rust_comments(text if text is not None else rust_source("lib.rs"))
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[[^\]]*\]\s*)*pub struct (\w+)\s*\{(.*?)\}", text, flags=re.S):
        fields = [(f, " ".join(t.split())) for f, t in re.findall(r"pub (\w+):\s*([^,]+),", m.group(2))]
        out[m.group(1)] = fields
    return out


def rust_functions(text=None):
    text = strip_rust_comments(text if text is not None else rust_source("lib.rs"))
    block = re.search(r'extern "C"\s*\{(.*?)\n\}', text, flags=re.S)
    assert block, 'no extern "C" block'
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block.group(1), flags=re.S):
        params = []
        for a in m.group(2).split(","):
            a = " ".join(a.split())
            if not a:
                continue
            name, ty = a.split(":", 1)
            params.append((name.strip(), ty.strip()))
        out[m.group(1)] = (params, (m.group(3) or "()").strip())
    return out


def rust_consts():
    text = strip_rust_comments(rust_source("lib.rs"))
    return dict(re.findall(r"pub const (ST_[A-Z_]+):\s*\w+\s*=\s*([^;]+);", text))


def size_of(rust_type, structs):
    if rust_type.startswith("*"):
        return 8, 8
    if rust_type in structs:
        off, align = 0, 1
        for _, t in structs[rust_type]:
            s, a = size_of(t, structs)
            off = (off + a - 1) // a * a + s
            align = max(align, a)
        return (off + align - 1) // align * align, align
    s = SIZES[rust_type]
    return s, s


def test_crate_files_exist():
    for rel in ["Cargo.toml", "build.rs", "src/lib.rs", "src/safe.rs"]:
        assert os.path.isfile(os.path.join(CRATE, rel)), rel
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert re.search(r'^name\s*=\s*"scratchtape-hip-sys"', cargo, flags=re.M)
    assert re.search(r'^links\s*=\s*"scratchtape_hip"', cargo, flags=re.M)
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "cargo:rustc-link-lib=dylib=scratchtape_hip" in build
    assert "SCRATCHTAPE_HIP_DIR" in build


def test_structs_match_the_header_field_for_field():
    want, got = header_structs(), rust_structs()
    assert set(want) == {"st_matref", "st_epilogue", "st_gemm"}
    assert set(got) == set(want)
    for name in want:
        assert got[name] == want[name], name


def test_struct_sizes_match_the_ctypes_binding():
    structs = rust_structs()
    from scratchtape_amd import _lib
    import ctypes
    for name, ct in [("st_matref", _lib.StMatRef), ("st_epilogue", _lib.StEpilogue), ("st_gemm", _lib.StGemm)]:
        assert size_of(name, structs)[0] == ctypes.sizeof(ct), name
    assert [size_of(n, structs)[0] for n in ("st_matref", "st_epilogue", "st_gemm")] == [56, 88, 296]


def test_extern_block_declares_exactly_the_header_functions():
    want, got = header_functions(), rust_functions()
    assert len(want) >= 29
    assert set(got) == set(want), (set(want) ^ set(got))
    for name, (params, ret) in want.items():
        rparams, rret = got[name]
        assert rparams == params, name
        assert rret == ret, name


def test_constants_match_the_header():
    defines, consts = header_defines(), rust_consts()
    for name in ["ST_OK", "ST_ERR_INVALID", "ST_ERR_HIP", "ST_ERR_OOM", "ST_ERR_NO_DEVICE"]:
        assert int(consts[name]) == int(defines[name].strip("()")), name
    c_bytes = eval(defines["ST_NOALLOC_SCRATCH_BYTES"].replace("u", ""))  # "(64u << 20)"
    assert eval(consts["ST_NOALLOC_SCRATCH_BYTES"]) == c_bytes


def test_safe_wrappers_call_only_declared_functions():
    declared = set(rust_functions())
    called = set(re.findall(r"sys::(st_[a-z0-9_]+)\s*\(", strip_rust_comments(rust_source("safe.rs"))))
    assert called and called <= declared, called - declared
    # the reference's matmul entry points, NdArray::matmul, LayerNorm and the kNN search all have one
    for name in ["st_matmul", "st_matmul_f32", "st_matmul_with", "st_matmul_grouped", "st_ndarray_matmul",
                 "st_layer_norm", "st_layer_norm_backward", "st_knn_probe", "st_knn_search_ivf_2bit",
                 "st_knn_search_masked_2bit"]:
        assert name in called, name


def test_safe_wrappers_define_their_helpers():
    text = strip_rust_comments(rust_source("safe.rs"))
    for helper in ["handle_ptr", "dptr", "ptr", "stream", "set_stream"]:
        assert re.search(rf"pub fn {helper}\b", text), helper
    # the reference's assert messages of NdArray::matmul (tensor.rs:249-253) are kept
    for msg in ["matmul lhs must be 2D", "matmul rhs must be 2D", "matmul inner dims must match"]:
        assert msg in text


PLANTS = {
    # two fields of st_epilogue swapped
    "swap": ("    pub bias_off: i64,\n    pub bias_stride: i64,", "    pub bias_stride: i64,\n    pub bias_off: i64,"),
    # a field's type changed
    "type": ("    pub relu: i32,", "    pub relu: i64,"),
    # a parameter's pointer constness flipped
    "const": ("dy: *const f32,\n        y: *const f32,", "dy: *mut f32,\n        y: *const f32,"),
    # a declaration dropped
    "drop": ("    pub fn st_sync(stream: st_stream) -> st_status;\n", ""),
}


@pytest.mark.parametrize("planted", sorted(PLANTS))
def test_the_checks_catch_a_planted_mismatch(planted):
    """The comparisons are not vacuous: each planted edit of lib.rs makes one of them fail."""
    old, new = PLANTS[planted]
    text = rust_source("lib.rs")
    assert text.count(old) == 1, planted
    bad = text.replace(old, new)
    structs_ok = rust_structs(bad) == header_structs()
    funcs_ok = rust_functions(bad) == header_functions()
    assert not (structs_ok and funcs_ok), planted
