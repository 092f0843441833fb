"""The Rust crate (crates/hip-bridge) declares the C ABI exactly as
include/hip_bridge.h does (no GPU, no Rust toolchain needed): every entry
point, with the same argument count, and each argument and return value of
the same type, pointer depth and constness; the #[repr(C)] structs have the
header's fields in the header's order and types; the status codes agree.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hip_bridge.h")
CRATE = os.path.join(ROOT, "crates", "hip-bridge")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")

C_BASE = {"int": "i32", "int32_t": "i32", "uint32_t": "u32", "uint64_t": "u64", "uint16_t": "u16",
          "float": "f32", "double": "f64", "char": "c_char", "void": "c_void"}
RUST_BASE = {"c_int": "i32", "i32": "i32", "u32": "u32", "u64": "u64", "u16": "u16", "f32": "f32",
             "f64": "f64", "c_char": "c_char", "c_void": "c_void"}


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def c_type(decl):
    """'const float* wq' -> '*const f32'; 'hb_ctx** out' -> '*mut *mut hb_ctx'; 'int B' -> 'i32'."""
    decl = decl.strip()
    depth = decl.count("*")
    words = decl.replace("*", " ").split()
    const = "const" in words
    words = [w for w in words if w != "const"]
    base = words[0]
    base = C_BASE.get(base, base)
    if depth == 0:
        return base
    out = ("*const " if const else "*mut ") + base
    for _ in range(depth - 1):
        out = "*mut " + out
    return out


def rust_type(t):
    t = " ".join(t.replace("*", " * ").split())
    parts = t.split()
    ptrs = []
    i = 0
    while parts[i] == "*":
        ptrs.append(parts[i + 1])  # const | mut
        i += 2
    base = "".join(parts[i:])
    base = RUST_BASE.get(base, base)
    for q in reversed(ptrs):
        base = f"*{q} {base}"
    return base


def header_prototypes():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(hb_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        ret = ret.split("\n")[-1].strip()
        params = [] if args in ("", "void") else [c_type(a) for a in args.split(",")]
        out[name] = (c_type(ret + " x") if "*" in ret else C_BASE.get(ret.split()[-1], ret), params)
    return out


def header_structs():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"typedef struct (hb_\w+) \{(.*?)\} \1;", text, flags=re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = decl.strip()
            if not decl:
                continue
            ty, names = decl.split(None, 1) if "*" not in decl else (decl.split("*")[0] + "*", decl.split("*")[1])
            for n in names.split(","):
                fields.append((n.strip(), c_type(ty)))
        out[m.group(1)] = fields
    return out


def rust_source():
    text = open(LIB_RS).read()
    return re.sub(r"//[^\n]*", "", text)


def rust_prototypes():
    text = rust_source()
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (hb_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        name, args, ret = m.group(1), m.group(2), (m.group(3) or "()").strip()
        params = [rust_type(a.split(":", 1)[1]) for a in args.split(",") if a.strip()]
        out[name] = (rust_type(ret), params)
    return out


def rust_structs():
    text = rust_source()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\][^\n]*\n(?:\s*#\[[^\n]*\n)*\s*pub struct (hb_\w+) \{(.*?)\}", text, flags=re.S):
        fields = []
        for line in m.group(2).split(","):
            line = line.strip()
            if line.startswith("pub "):
                n, t = line[4:].split(":", 1)
                fields.append((n.strip(), rust_type(t)))
        out[m.group(1)] = fields
    return out


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.isfile(os.path.join(CRATE, f)), f
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "hip-bridge"' in toml and 'links = "hip_bridge"' in toml
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=hip_bridge" in build


def test_every_header_entry_point_is_declared_with_the_same_signature():
    hdr, rs = header_prototypes(), rust_prototypes()
    assert len(hdr) > 60
    assert sorted(hdr) == sorted(rs), (sorted(set(hdr) ^ set(rs)))
    bad = []
    for name, (ret, params) in hdr.items():
        rret, rparams = rs[name]
        if ret != rret or params != rparams:
            bad.append((name, (ret, params), (rret, rparams)))
    assert not bad, bad


def test_structs_match_the_header_field_for_field():
    hdr, rs = header_structs(), rust_structs()
    assert set(hdr) == {"hb_model_config", "hb_train_config", "hb_forward_result", "hb_forward_timings",
                        "hb_rstk_header"}
    for name, fields in hdr.items():
        assert rs.get(name) == fields, (name, fields, rs.get(name))


def test_status_codes_and_constants_agree():
    text = _strip_c_comments(open(HEADER).read())
    codes = dict((n, int(v)) for n, v in re.findall(r"\b(HB_(?:OK|E_\w+|DTYPE_F16))\s*=\s*(-?\d+)", text))
    rs = rust_source()
    for n, v in codes.items():
        m = re.search(rf"pub const {n}: c_int = (-?\d+);", rs)
        assert m and int(m.group(1)) == v, n
    assert "HB_SYNTH_EMBED_ID: u64 = 0xFFFF" in rs and "HB_SYNTH_EMBED_ID 0xFFFFu" in text


@pytest.mark.parametrize("planted", ["drop_arg", "const_flip", "rename"])
def test_the_check_catches_planted_mistakes(planted, monkeypatch):
    """A binding with one argument dropped, one constness flipped or one
    function renamed must fail the signature comparison."""
    src = open(LIB_RS).read()
    if planted == "drop_arg":
        bad = src.replace("pub fn hb_model_reserve(model: *mut hb_model, b: c_int, s: c_int)",
                          "pub fn hb_model_reserve(model: *mut hb_model, b: c_int)")
    elif planted == "const_flip":
        bad = src.replace("pub fn hb_tokens_length(t: *const hb_tokens", "pub fn hb_tokens_length(t: *mut hb_tokens")
    else:
        bad = src.replace("pub fn hb_kv_reset(", "pub fn hb_kv_clear(")
    assert bad != src
    import sys
    monkeypatch.setattr(sys.modules[__name__], "rust_source", lambda: re.sub(r"//[^\n]*", "", bad))
    with pytest.raises(AssertionError):
        test_every_header_entry_point_is_declared_with_the_same_signature()
