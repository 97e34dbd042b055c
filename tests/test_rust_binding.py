"""CPU: the Rust binding (emel.rs_amd/rust/emel-kernels-hip) against
include/emel_hip.h.

This environment has no Rust toolchain, so the crate is never compiled
here.  These checks are what stands in for it, and they cover exactly what
a wrong binding breaks silently at run time:

  * every function the header declares is in the crate's `extern "C"` block
    with the same parameter names, order and types and the same return
    type, and nothing else is;
  * every struct has the same fields in the same order with the same Rust
    equivalent types, and the `#[repr(C)]` layout computed from the Rust
    field types (size/alignment rules of x86-64) equals the C layout that
    gcc reports for the header (`offsetof` / `sizeof` of every field);
  * every enum constant has the value gcc gives it;
  * the safe layer calls only declared functions, and reaches all of them.

A Rust type error inside the safe layer is not caught here; brackets and
module files are checked for balance and presence only.
"""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "emel_hip.h"
CRATE = ROOT / "emel.rs_amd" / "rust" / "emel-kernels-hip"
FFI = CRATE / "src" / "ffi.rs"

RUST_KEYWORDS = {"in", "type", "ref", "mod", "fn", "match", "loop", "move", "self", "use", "impl",
                 "where", "struct", "enum", "mut", "const", "static", "trait", "unsafe", "extern"}

# C type of a parameter / field / return value -> its Rust equivalent.
C_TO_RUST = {
    "const void *": "*const c_void",
    "void *": "*mut c_void",
    "void **": "*mut *mut c_void",
    "const float *": "*const f32",
    "float *": "*mut f32",
    "const int32_t *": "*const i32",
    "int32_t *": "*mut i32",
    "uint32_t *": "*mut u32",
    "uint64_t *": "*mut u64",
    "const char *": "*const c_char",
    "uint8_t": "u8",
    "uint32_t": "u32",
    "int32_t": "i32",
    "uint64_t": "u64",
    "float": "f32",
    "emel_status": "Status",
    "emel_stream": "Stream",
    "emel_stream *": "*mut Stream",
    # enum-typed parameters travel as their 32-bit code
    "emel_unary_subop": "u32",
    "emel_binary_op": "u32",
    "emel_glu_subop": "u32",
}

# Size and alignment of each Rust field type on x86-64.
RUST_SCALARS = {"u8": 1, "u32": 4, "i32": 4, "f32": 4, "u64": 8}


def strip_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def norm_c(ty):
    ty = " ".join(ty.split())
    ty = re.sub(r"\s*\*\s*", "*", ty)
    ty = re.sub(r"(\w)\*", r"\1 *", ty)
    return ty


def camel(name):
    return "".join(part.capitalize() for part in name.split("_"))


def c_to_rust(ty):
    ty = norm_c(ty)
    if ty in C_TO_RUST:
        return C_TO_RUST[ty]
    m = re.fullmatch(r"const (emel_\w+) \*", ty)
    assert m, f"no Rust equivalent recorded for C type {ty!r}"
    return "*const " + camel(m.group(1))


# ---- header side -------------------------------------------------------------------

def header_functions():
    text = strip_comments(HEADER.read_text())
    out = {}
    pat = r"^\s*((?:const\s+)?\w+\s*\**)\s*(emel_\w+)\s*\(([^;]*?)\)\s*;"
    for m in re.finditer(pat, text, flags=re.M | re.S):
        args = " ".join(m.group(3).split())
        params = []
        if args not in ("", "void"):
            for p in args.split(","):
                pm = re.fullmatch(r"(.*?)(\w+)", p.strip())
                params.append((pm.group(2), norm_c(pm.group(1))))
        out[m.group(2)] = (norm_c(m.group(1)), params)
    return out


def header_structs():
    text = strip_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"typedef struct (\w+)\s*\{(.*?)\}\s*\w+\s*;", text, flags=re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            fm = re.fullmatch(r"(.*?)(\w+)(?:\[(\d+)\])?", decl)
            fields.append((fm.group(2), norm_c(fm.group(1)), int(fm.group(3)) if fm.group(3) else None))
        out[m.group(1)] = fields
    return out


def header_enum_names():
    text = strip_comments(HEADER.read_text())
    names = []
    for m in re.finditer(r"typedef enum (\w+)\s*\{(.*?)\}\s*\w+\s*;", text, flags=re.S):
        for entry in m.group(2).split(","):
            entry = entry.strip()
            if entry:
                names.append(re.match(r"\w+", entry).group(0))
    return names


@pytest.fixture(scope="module")
def c_facts(tmp_path_factory):
    """sizeof/offsetof of every header struct field and the value of every
    enum constant, as gcc compiles the header."""
    structs = header_structs()
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for name, fields in structs.items():
        lines.append(f'printf("S {name} %zu %zu\\n", sizeof({name}), _Alignof({name}));')
        for fname, _, _ in fields:
            lines.append(f'printf("F {name} {fname} %zu %zu\\n", offsetof({name}, {fname}), '
                         f'sizeof((({name} *)0)->{fname}));')
    for const in header_enum_names():
        lines.append(f'printf("E {const} %lld\\n", (long long){const});')
    lines += ["return 0;", "}"]
    work = tmp_path_factory.mktemp("cfacts")
    src, exe = work / "facts.c", work / "facts"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-o", str(exe), str(src)], check=True)
    facts = {"S": {}, "F": {}, "E": {}}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        kind, *rest = line.split()
        if kind == "S":
            facts["S"][rest[0]] = (int(rest[1]), int(rest[2]))
        elif kind == "F":
            facts["F"][(rest[0], rest[1])] = (int(rest[2]), int(rest[3]))
        else:
            facts["E"][rest[0]] = int(rest[1])
    return facts


# ---- Rust side -----------------------------------------------------------------------

def rust_source():
    return re.sub(r"//[^\n]*", "", FFI.read_text())


def rust_externs():
    text = rust_source()
    block = re.search(r'unsafe extern "C"\s*\{(.*?)\n\}', text, flags=re.S)
    assert block, "ffi.rs has no unsafe extern \"C\" block"
    out = {}
    for m in re.finditer(r"pub fn (\w+)\((.*?)\)\s*->\s*([^;]+);", block.group(1), flags=re.S):
        params = []
        args = " ".join(m.group(2).split())
        if args:
            for p in args.split(","):
                pname, pty = (s.strip() for s in p.split(":", 1))
                params.append((pname, " ".join(pty.split())))
        assert m.group(1) not in out, f"{m.group(1)} declared twice"
        out[m.group(1)] = (" ".join(m.group(3).split()), params)
    return out


def rust_structs():
    text = rust_source()
    out = {}
    for m in re.finditer(r"(#\[repr\(C\)\]\s*(?:#\[[^\]]*\]\s*)*)pub struct (\w+)\s*\{(.*?)\}", text, flags=re.S):
        fields = []
        for decl in m.group(3).split(","):
            decl = " ".join(decl.split())
            if decl:
                fm = re.fullmatch(r"pub (\w+): (.+)", decl)
                assert fm, f"unparsed field {decl!r} in {m.group(2)}"
                fields.append((fm.group(1), fm.group(2)))
        out[m.group(2)] = fields
    # every pub struct must be repr(C)
    assert len(out) == len(re.findall(r"pub struct \w+", text))
    return out


def rust_consts():
    text = rust_source()
    return {m.group(1): (m.group(2), int(m.group(3)))
            for m in re.finditer(r"pub const (\w+): (\w+) = (\d+);", text)}


def rust_type_layout(ty):
    """(size, align) of a Rust field type under repr(C) on x86-64."""
    arr = re.fullmatch(r"\[(.+); (\d+)\]", ty)
    if arr:
        size, align = rust_type_layout(arr.group(1))
        return size * int(arr.group(2)), align
    if ty.startswith("*const ") or ty.startswith("*mut "):
        return 8, 8
    assert ty in RUST_SCALARS, f"unknown Rust field type {ty!r}"
    return RUST_SCALARS[ty], RUST_SCALARS[ty]


def repr_c_layout(fields):
    offset, align, offsets = 0, 1, {}
    for name, ty in fields:
        size, a = rust_type_layout(ty)
        offset = (offset + a - 1) // a * a
        offsets[name] = (offset, size)
        offset += size
        align = max(align, a)
    return offsets, (offset + align - 1) // align * align, align


# ---- tests ---------------------------------------------------------------------------------

def test_crate_files_present():
    for rel in ["Cargo.toml", "build.rs", "src/lib.rs", "src/ffi.rs", "src/event.rs", "src/graph.rs"]:
        assert (CRATE / rel).is_file(), rel
    lib = (CRATE / "src" / "lib.rs").read_text()
    for mod in re.findall(r"^\s*(?:pub )?mod (\w+);", lib, flags=re.M):
        assert (CRATE / "src" / f"{mod}.rs").is_file(), f"module {mod} has no file"


def test_every_header_function_is_bound_with_its_signature():
    header, rust = header_functions(), rust_externs()
    assert len(header) >= 70
    assert sorted(header) == sorted(rust), (set(header) ^ set(rust))
    for name, (cret, cparams) in header.items():
        rret, rparams = rust[name]
        assert rret == c_to_rust(cret), (name, cret, rret)
        assert len(rparams) == len(cparams), name
        for (cn, cty), (rn, rty) in zip(cparams, rparams):
            expect_name = cn + "_" if cn in RUST_KEYWORDS else cn
            assert rn == expect_name, (name, cn, rn)
            assert rty == c_to_rust(cty), (name, cn, cty, rty)


def test_struct_fields_match_in_order_and_type():
    header, rust = header_structs(), rust_structs()
    assert sorted(camel(n) for n in header) == sorted(rust)
    for cname, cfields in header.items():
        rfields = rust[camel(cname)]
        assert [f[0] for f in rfields] == [f[0] for f in cfields], cname
        for (fname, cty, n), (_, rty) in zip(cfields, rfields):
            expect = c_to_rust(cty)
            if n is not None:
                expect = f"[{expect}; {n}]"
            assert rty == expect, (cname, fname, cty, rty)


def test_repr_c_layout_equals_gcc_layout(c_facts):
    header, rust = header_structs(), rust_structs()
    for cname in header:
        offsets, size, align = repr_c_layout(rust[camel(cname)])
        assert (size, align) == c_facts["S"][cname], cname
        for fname, (off, fsize) in offsets.items():
            assert (off, fsize) == c_facts["F"][(cname, fname)], (cname, fname)


def test_enum_constants_have_gcc_values(c_facts):
    consts = rust_consts()
    assert len(c_facts["E"]) >= 150
    for name, value in c_facts["E"].items():
        assert name in consts, f"{name} missing from ffi.rs"
        rty, rvalue = consts[name]
        assert rvalue == value, (name, value, rvalue)
        assert rty == ("Status" if name.startswith(("EMEL_OK", "EMEL_ERR_")) else "u32"), name
    abi = re.search(r"#define EMEL_HIP_ABI_VERSION (\d+)u", HEADER.read_text()).group(1)
    assert consts["EMEL_HIP_ABI_VERSION"][1] == int(abi)
    inline = re.search(r"#define EMEL_GET_ROWS_INLINE_INDICES (\d+)u", HEADER.read_text()).group(1)
    assert consts["EMEL_GET_ROWS_INLINE_INDICES"][1] == int(inline)


def test_safe_layer_calls_only_declared_functions_and_all_of_them():
    declared = set(rust_externs())
    used = set()
    for path in (CRATE / "src").glob("*.rs"):
        if path.name == "ffi.rs":
            continue
        used |= set(re.findall(r"ffi::(emel_\w+)", path.read_text()))
    assert used <= declared, used - declared
    assert declared <= used, f"no safe wrapper for {sorted(declared - used)}"


def test_sources_balance_brackets():
    for path in list((CRATE / "src").glob("*.rs")) + [CRATE / "build.rs"]:
        text = path.read_text()
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r'"(?:\\.|[^"\\])*"', '""', text)
        text = re.sub(r"'(?:\\.|[^'\\])'", "''", text)
        for open_, close in ["{}", "()", "[]"]:
            assert text.count(open_) == text.count(close), (path.name, open_)
