"""The Rust FFI crate (crates/diffrast-hip) against include/diffrast_hip.h.

No Rust toolchain exists in this image, so the crate is checked by parsing:
every C function has an `extern "C"` declaration with the same name, arity,
parameter names and types (mapped C -> Rust); every C struct a `#[repr(C)]`
struct with the same fields in the same order and types; every status code,
flag and enum value the same constant. The safe wrapper's calls into `ffi::`
name declared functions with the declared number of arguments.
"""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "diffrast_hip.h"
CRATE = ROOT / "crates" / "diffrast-hip"
FFI = CRATE / "src" / "ffi.rs"
LIB = CRATE / "src" / "lib.rs"

C_BASE = {
    "float": "f32", "double": "f64", "int": "c_int", "int32_t": "i32", "int64_t": "i64",
    "uint8_t": "u8", "uint32_t": "u32", "uint64_t": "u64", "size_t": "usize", "char": "c_char",
    "void": "c_void",
}


def c_to_rust(ctype: str) -> str:
    """`const float *` -> `*const f32`, `drh_ctx **` -> `*mut *mut drh_ctx`."""
    ctype = " ".join(ctype.replace("*", " * ").split())
    stars = ctype.count("*")
    words = ctype.replace("*", "").split()
    const = "const" in words
    base = [w for w in words if w != "const"]
    assert len(base) == 1, ctype
    rust = C_BASE.get(base[0], base[0])
    for level in range(stars):
        rust = ("*const " if (level == 0 and const) else "*mut ") + rust
    return rust


def strip_c_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def header_functions() -> dict:
    text = strip_c_comments(HEADER.read_text())
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(drh_\w+)\s*\(([^)]*)\)\s*;", text):
        params = []
        for a in args.split(","):
            a = " ".join(a.split())
            if not a or a == "void":
                continue
            m = re.match(r"(.*?)(\w+)$", a)
            params.append((m.group(2).lower(), c_to_rust(m.group(1))))
        ret = ret.strip().split("\n")[-1].strip()
        out[name] = (params, c_to_rust(ret))
    return out


def header_structs() -> dict:
    text = strip_c_comments(HEADER.read_text())
    out = {}
    for body, name in re.findall(r"typedef struct\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.match(r"([\w\s\*]+?)\s+(\w+(?:\s*,\s*\w+)*)$", decl)
            ctype, names = m.group(1), m.group(2)
            for n in names.split(","):
                fields.append((n.strip(), c_to_rust(ctype)))
        out[name] = fields
    for name in re.findall(r"typedef struct (\w+) \1\s*;", text):
        out[name] = None  # opaque
    return out


def header_constants() -> dict:
    text = strip_c_comments(HEADER.read_text())
    out = {}
    for name, val in re.findall(r"#define\s+(DRH_\w+)\s+(0x[0-9a-fA-F]+|\d+)u?\b", text):
        out[name] = int(val, 0)
    for body in re.findall(r"enum\s*\{(.*?)\}", text, flags=re.S):
        for name, val in re.findall(r"(DRH_\w+)\s*=\s*(\d+)", body):
            out[name] = int(val)
    return out


def rust_source(path: Path) -> str:
    return re.sub(r"//[^\n]*", "", path.read_text())


def split_top(args: str) -> list:
    """Split on commas outside brackets and braces."""
    parts, depth, cur = [], 0, []
    for ch in args:
        if ch in "([{<":
            depth += 1
        elif ch in ")]}>":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append("".join(cur))
            cur = []
        else:
            cur.append(ch)
    parts.append("".join(cur))
    return [p.strip() for p in parts if p.strip()]


def rust_functions() -> dict:
    text = rust_source(FFI)
    block = re.search(r'extern "C"\s*\{(.*)\}', text, flags=re.S).group(1)
    out = {}
    for name, args, ret in re.findall(r"pub fn (\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, flags=re.S):
        params = []
        for a in split_top(args):
            pname, ptype = a.split(":", 1)
            params.append((pname.strip(), " ".join(ptype.split())))
        out[name] = (params, " ".join(ret.split()) if ret else "()")
    return out


def rust_structs() -> dict:
    text = rust_source(FFI)
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*(?:#\[derive\([^\]]*\)\]\s*)?pub struct (\w+)\s*\{(.*?)\}",
                                 text, flags=re.S):
        fields = []
        for f in split_top(body):
            m = re.match(r"(?:pub\s+)?(\w+)\s*:\s*(.+)$", " ".join(f.split()))
            fields.append((m.group(1), m.group(2)))
        out[name] = fields
    return out


def rust_constants() -> dict:
    text = rust_source(FFI)
    return {n: int(v, 0) for n, v in re.findall(r"pub const (DRH_\w+)\s*:\s*\w+\s*=\s*(0x[0-9a-fA-F]+|\d+)\s*;", text)}


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", "src/ffi.rs", "src/lib.rs"):
        assert (CRATE / f).is_file(), f
    toml = (CRATE / "Cargo.toml").read_text()
    assert 'name = "diffrast-hip"' in toml and 'links = "diffrast_hip"' in toml
    assert "rustc-link-lib=dylib=diffrast_hip" in (CRATE / "build.rs").read_text()


def test_the_type_mapping_itself():
    assert c_to_rust("const float *") == "*const f32"
    assert c_to_rust("drh_ctx **") == "*mut *mut drh_ctx"
    assert c_to_rust("const drh_ctx *") == "*const drh_ctx"
    assert c_to_rust("void *") == "*mut c_void"
    assert c_to_rust("int64_t") == "i64"


def test_every_function_is_declared_with_the_same_signature():
    c, rust = header_functions(), rust_functions()
    # the parser sees every symbol the header declares
    declared = set(re.findall(r"\b(drh_\w+)\s*\(", strip_c_comments(HEADER.read_text())))
    assert set(c) == declared, declared ^ set(c)
    assert sorted(c) == sorted(rust), set(c) ^ set(rust)
    for name, (cparams, cret) in c.items():
        rparams, rret = rust[name]
        assert len(rparams) == len(cparams), f"{name}: arity {len(rparams)} != {len(cparams)}"
        for i, ((cn, ct), (rn, rt)) in enumerate(zip(cparams, rparams)):
            assert rn == cn, f"{name} parameter {i}: {rn} != {cn}"
            assert rt == ct, f"{name}({cn}): {rt} != {ct}"
        assert rret == cret, f"{name} returns {rret}, the header {cret}"


def test_every_struct_has_the_same_fields_in_order():
    c, rust = header_structs(), rust_structs()
    assert sorted(c) == sorted(rust), set(c) ^ set(rust)
    for name, cfields in c.items():
        if cfields is None:
            assert rust[name] == [("_opaque", "[u8; 0]")], name
        else:
            assert rust[name] == cfields, name


def test_every_constant_has_the_same_value():
    c, rust = header_constants(), rust_constants()
    assert len(c) >= 20
    assert c == rust, {k: (c.get(k), rust.get(k)) for k in set(c) | set(rust) if c.get(k) != rust.get(k)}


def test_the_safe_wrapper_calls_declared_functions_with_their_arity():
    decl = rust_functions()
    text = rust_source(LIB)
    calls = 0
    for m in re.finditer(r"ffi::(drh_\w+)\s*\(", text):
        name = m.group(1)
        assert name in decl, name
        depth, i = 1, m.end()
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        args = split_top(text[m.end():i - 1])
        assert len(args) == len(decl[name][0]), f"{name}: {len(args)} arguments, declared {len(decl[name][0])}"
        calls += 1
    assert calls >= 20
    # every ffi constant and type the wrapper names exists
    consts, structs = rust_constants(), rust_structs()
    for name in set(re.findall(r"ffi::(DRH_\w+)", text)):
        assert name in consts, name
    for name in set(re.findall(r"ffi::(drh_[a-z_]+)\b(?!\s*\()", text)):
        assert name in structs, name


REFERENCE_GPU_METHODS = [  # crates/diffrast-gpu/src/lib.rs:232-910
    "new", "pool_stats", "clear_pool", "adapter_info", "is_discrete", "tape_bytes", "render", "backward",
    "backward_with", "render_many", "backward_many", "backward_many_timed", "backward_many_full",
    "backward_many_from_grad",
]
REFERENCE_FREE_FUNCTIONS = ["render", "render_batch", "render_with_tape", "backward", "backward_batch", "fit"]
REFERENCE_FITTER_METHODS = [  # crates/diffrast/src/fit.rs:214-334
    "new", "step", "scene", "target", "iter", "losses", "best_loss", "is_done", "sigma", "render_current",
    "into_report",
]


@pytest.mark.parametrize("kind", ["GpuRasterizer", "Fitter", "free"])
def test_the_wrapper_mirrors_the_reference_api(kind):
    text = rust_source(LIB)
    impls = re.split(r"\nimpl\b", text)
    if kind == "free":
        have = set(re.findall(r"^pub fn (\w+)", text, flags=re.M))
        want = REFERENCE_FREE_FUNCTIONS
    else:
        body = "\n".join(b for b in impls if re.match(rf"(<'\w+>)?\s*{kind}\b", b.strip()))
        have = set(re.findall(r"pub fn (\w+)", body))
        want = REFERENCE_GPU_METHODS if kind == "GpuRasterizer" else REFERENCE_FITTER_METHODS
    missing = [m for m in want if m not in have]
    assert not missing, missing
    for ty in ("GpuError", "ReduceMode", "BackwardMode", "BackwardTimings", "PoolStats", "BatchGradients"):
        assert re.search(rf"pub (enum|struct|type) {ty}\b", text), ty
