"""crates/hip/src/ffi.rs against include/linalg_hip.h (CPU only; there is no Rust toolchain here).

The Rust crate a maintainer adds to the reference (crates/hip) binds the C ABI through
src/ffi.rs. Every function the header declares must appear there under the same name with the
same number of parameters and the same C types in the same order and the same return type, and
the reverse; the four descriptor structs must have the same fields in the same order with the
same types and array lengths; the enum constants must have the header's values.
"""
from __future__ import annotations

import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = (REPO / "include" / "linalg_hip.h").read_text()
FFI = (REPO / "crates" / "hip" / "src" / "ffi.rs").read_text()

C_BASE = {"float": "f32", "int32_t": "i32", "uint32_t": "u32", "uint64_t": "u64", "uint8_t": "u8",
          "char": "c_char", "void": "c_void"}


def strip_c_comments(text: str) -> str:
    """The header without comments and preprocessor lines."""
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return re.sub(r"^\s*#[^\n]*", " ", text, flags=re.M)


def c_type(decl: str) -> str:
    """A C parameter or return declaration (name removed) in Rust spelling."""
    decl = " ".join(decl.split())
    array = decl.endswith("]")
    decl = re.sub(r"\[[^\]]*\]$", "", decl).strip()
    const = decl.startswith("const ")
    if const:
        decl = decl[len("const "):]
    stars = decl.count("*") + (1 if array else 0)
    base = decl.replace("*", "").strip()
    base = C_BASE.get(base, base)
    if stars == 0:
        return base
    out = ("*const " if const else "*mut ") + base
    for _ in range(stars - 1):
        out = "*mut " + out
    return out


def c_param(p: str) -> str:
    p = " ".join(p.split())
    m = re.match(r"^(.*?)(\w+)(\s*\[[^\]]*\])?$", p)
    assert m, p
    return c_type(m.group(1) + (m.group(3) or ""))


def header_functions() -> dict:
    text = strip_c_comments(HEADER)
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(lg_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ret = " ".join(ret.split())
        ps = [] if params.strip() in ("", "void") else [c_param(p) for p in params.split(",")]
        out[name] = (None if ret == "void" else c_type(ret), ps)
    return out


def ffi_functions() -> dict:
    block = FFI[FFI.index('extern "C" {'):]
    block = re.sub(r"//[^\n]*", " ", block)
    out = {}
    for m in re.finditer(r"pub fn (lg_\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        ps = []
        for p in params.split(","):
            if p.strip():
                ps.append(" ".join(p.split(":", 1)[1].split()))
        out[name] = (None if ret is None else " ".join(ret.split()), ps)
    return out


def header_structs() -> dict:
    text = strip_c_comments(HEADER)
    out = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} \1;", text, flags=re.S):
        fields = []
        for f in m.group(2).split(";"):
            f = " ".join(f.split())
            if not f:
                continue
            # "uint64_t batch, m, n, k" declares four fields of one type.
            first, *more = [x.strip() for x in f.split(",")]
            fm = re.match(r"^(.*?)(\w+)(\[([^\]]+)\])?$", first)
            ty = c_type(fm.group(1))
            fields.append((fm.group(2), ty, fm.group(4)))
            for name in more:
                am = re.match(r"^(\w+)(\[([^\]]+)\])?$", name)
                fields.append((am.group(1), ty, am.group(3)))
        out[m.group(1)] = fields
    return out


def ffi_structs() -> dict:
    out = {}
    for m in re.finditer(r"pub struct (lg_\w+) \{(.*?)\}", FFI, flags=re.S):
        fields = []
        for f in m.group(2).split(","):
            f = " ".join(f.split())
            if not f.startswith("pub "):
                continue
            name, ty = f[len("pub "):].split(":", 1)
            ty = ty.strip()
            am = re.match(r"^\[(\S+); (\S+)\]$", ty)
            fields.append((name.strip(), am.group(1), am.group(2)) if am else (name.strip(), ty, None))
        out[m.group(1)] = fields
    return out


def test_every_header_function_is_bound_with_the_same_signature():
    from linalg_hip import _native as N
    h, r = header_functions(), ffi_functions()
    # The same set the library exports and the Python binding declares.
    assert set(h) == set(N.SIGNATURES), set(h) ^ set(N.SIGNATURES)
    assert set(h) == set(r), {"header only": sorted(set(h) - set(r)), "ffi only": sorted(set(r) - set(h))}
    for name in sorted(h):
        assert len(h[name][1]) == len(r[name][1]), (name, h[name], r[name])
        assert h[name] == r[name], (name, h[name], r[name])


def test_descriptor_structs_match_field_for_field():
    h, r = header_structs(), ffi_structs()
    for name in ("lg_view", "lg_tensor", "lg_contract_plan", "lg_permute_plan"):
        assert h[name] == r[name], (name, h[name], r[name])


@pytest.mark.parametrize("enum", ["lg_status", "lg_elem", "lg_core_error", "lg_dtype"])
def test_enum_constants_match(enum):
    text = strip_c_comments(HEADER)
    body = re.search(r"typedef enum %s \{(.*?)\} %s;" % (enum, enum), text, flags=re.S).group(1)
    consts = dict((k.strip(), int(v)) for k, v in re.findall(r"(\w+)\s*=\s*(\d+)", body))
    rust = dict((k, int(v)) for k, v in re.findall(r"pub const (\w+): %s = (\d+);" % enum, FFI))
    assert consts == rust, (enum, consts, rust)


def test_the_parsers_see_a_planted_mismatch():
    """A changed parameter type or a dropped parameter in the Rust text must be caught."""
    r = ffi_functions()
    h = header_functions()
    assert r["lg_gemm_f32"] == h["lg_gemm_f32"]
    bad = FFI.replace("pub fn lg_gemm_f32(ctx: *mut lg_ctx, alpha: f32,", "pub fn lg_gemm_f32(ctx: *mut lg_ctx, alpha: f64,")
    assert bad != FFI
    block = re.sub(r"//[^\n]*", " ", bad[bad.index('extern "C" {'):])
    m = re.search(r"pub fn lg_gemm_f32\s*\(([^)]*)\)", block)
    assert " ".join(m.group(1).split(",")[1].split(":", 1)[1].split()) == "f64" != h["lg_gemm_f32"][1][1]
