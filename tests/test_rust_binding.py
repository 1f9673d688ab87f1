"""The Rust FFI crate (falcon-ocr-cpu_amd/focr-hip-sys) against the C header.

No Rust toolchain exists in this image, so the crate is checked by parsing:
every function that include/focr_hip.h declares appears in the crate's
`extern "C"` block with the same name, the same number of arguments and the
same type for each of them (pointer depth, constness and pointee, integer and
float widths), and every FOCR_* constant has the header's value. A crate that
drifts from the header fails here before a maintainer's `cargo build` would
link it.
"""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "focr_hip.h"
CRATE = ROOT / "falcon-ocr-cpu_amd" / "focr-hip-sys"

C_BASE = {"int": "int", "size_t": "usize", "float": "f32", "void": "void", "char": "char", "int8_t": "i8",
          "int32_t": "i32", "uint32_t": "u32"}
RUST_BASE = {"c_int": "int", "usize": "usize", "f32": "f32", "c_void": "void", "c_char": "char", "i8": "i8",
             "i32": "i32", "u32": "u32"}


def c_type(text: str) -> str:
    """Canonical form of a C type (the parameter name already removed):
    pointer levels outermost first, e.g. `const float *` -> `*const f32`."""
    text = text.strip()
    stars = text.count("*")
    parts = re.split(r"(\*)", text)
    base_part = parts[0].split()
    const_base = "const" in base_part
    base = [t for t in base_part if t != "const"]
    assert len(base) == 1, text
    name = C_BASE.get(base[0], base[0])
    # Each '*' may be followed by `const` (a const pointer), which this ABI never uses.
    assert "const" not in "".join(parts[1:]), f"const pointer in {text!r}"
    out = name
    for level in range(stars):
        innermost = level == 0
        out = ("*const " if (innermost and const_base) else "*mut ") + out
    assert stars or not const_base, text
    return out


def split_c_param(param: str):
    param = param.strip()
    if param == "void":
        return None
    m = re.match(r"^(.*?)([A-Za-z_][A-Za-z0-9_]*)$", param)
    assert m, param
    return c_type(m.group(1))


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = "\n".join(line for line in text.splitlines() if not line.strip().startswith("#"))
    text = text.replace('extern "C" {', "")
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(focr_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        ret, name, params = m.group(1), m.group(2), " ".join(m.group(3).split())
        args = [split_c_param(p) for p in params.split(",")] if params.strip() else []
        args = [a for a in args if a is not None]
        out[name] = (c_type(ret), args)
    return out


def rust_type(text: str) -> str:
    text = " ".join(text.split())
    out = []
    while True:
        m = re.match(r"^\*(const|mut)\s+(.*)$", text)
        if not m:
            break
        out.append(f"*{m.group(1)} ")
        text = m.group(2)
    base = RUST_BASE.get(text, text)
    return "".join(out) + base


def crate_functions():
    text = (CRATE / "src" / "lib.rs").read_text()
    text = re.sub(r"//[^\n]*", "", text)
    block = re.search(r'extern "C"\s*\{(.*?)\n\}', text, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (focr_[a-z0-9_]+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        args = []
        for p in params.split(","):
            p = p.strip()
            if not p:
                continue
            _, ty = p.split(":", 1)
            args.append(rust_type(ty))
        out[name] = (rust_type(ret) if ret else "void", args)
    return out


def test_type_parser_on_known_forms():
    assert c_type("const float *") == "*const f32"
    assert c_type("focr_ctx **") == "*mut *mut focr_ctx"
    assert c_type("const focr_linear *") == "*const focr_linear"
    assert c_type("size_t") == "usize"
    assert rust_type("*mut *mut focr_ctx") == "*mut *mut focr_ctx"
    assert rust_type("*const c_char") == "*const char"


def test_every_header_function_is_bound_with_the_same_types():
    header, crate = header_functions(), crate_functions()
    assert len(header) >= 40, sorted(header)
    assert sorted(header) == sorted(crate), (sorted(set(header) ^ set(crate)))
    for name, (ret, args) in header.items():
        rret, rargs = crate[name]
        assert ret == rret, f"{name}: returns {ret} in C, {rret} in Rust"
        assert len(args) == len(rargs), f"{name}: {len(args)} arguments in C, {len(rargs)} in Rust"
        for i, (a, b) in enumerate(zip(args, rargs)):
            assert a == b, f"{name} argument {i}: {a} in C, {b} in Rust"


def test_constants_match_the_header():
    defines = dict(re.findall(r"#define (FOCR_[A-Z0-9_]+) \(?(-?\d+)\)?", HEADER.read_text()))
    rust = dict(re.findall(r"pub const (FOCR_[A-Z0-9_]+): c_int = (-?\d+);", (CRATE / "src" / "lib.rs").read_text()))
    assert defines and defines == rust


def test_crate_files_exist_and_link_the_library():
    manifest = (CRATE / "Cargo.toml").read_text()
    assert 'name = "focr-hip-sys"' in manifest and 'links = "focr_hip"' in manifest
    build = (CRATE / "build.rs").read_text()
    assert "rustc-link-lib=dylib=focr_hip" in build
