"""Writes src/ffi.rs, the Rust mirror of include/mamba_hip.h: one #[repr(C)]
struct per argument struct (same fields, same order), the status / dtype
constants, and one `extern "C"` declaration per entry point.

    python gen_ffi.py            # rewrite src/ffi.rs from the header
    python gen_ffi.py --check    # exit 1 if src/ffi.rs is out of date

The crate has no logic beyond this marshalling, so a header that changes is
followed by running this script; tests/test_rust_ffi.py checks the committed
file against the header and its layouts against the C compiler's."""

from __future__ import annotations

import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "..", "..", "include", "mamba_hip.h")
OUT = os.path.join(HERE, "src", "ffi.rs")

SCALARS = {"int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "int": "c_int", "size_t": "usize",
           "float": "f32", "double": "f64"}
RUST_KEYWORDS = {"as", "break", "const", "continue", "crate", "else", "enum", "extern", "false", "fn", "for", "if",
                 "impl", "in", "let", "loop", "match", "mod", "move", "mut", "pub", "ref", "return", "self", "Self",
                 "static", "struct", "super", "trait", "true", "type", "unsafe", "use", "where", "while", "async",
                 "await", "dyn"}


def camel(c_name: str) -> str:
    """mamba_ssd2_args -> MambaSsd2Args, mamba1_scan_args -> Mamba1ScanArgs."""
    return "".join(p[:1].upper() + p[1:] for p in c_name.split("_"))


def strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def rust_type(c_type: str, structs: set) -> str:
    """A C declaration's type (with its '*' and const) as the Rust FFI type."""
    t = " ".join(c_type.replace("*", " * ").split())
    if t == "mamba_stream_t":
        return "MambaStream"
    if t == "void * const *":
        return "*const *mut c_void"
    m = re.fullmatch(r"(const )?(\w+)( \*)?", t)
    if not m:
        raise ValueError(f"unsupported C type: {c_type!r}")
    const, base, ptr = m.groups()
    if base == "void":
        inner = "c_void"
    elif base == "char":
        inner = "c_char"
    elif base in SCALARS:
        inner = SCALARS[base]
    elif base in structs:
        inner = camel(base)
    else:
        raise ValueError(f"unknown C type: {c_type!r}")
    if ptr:
        return ("*const " if const else "*mut ") + inner
    return inner


def field_name(name: str) -> str:
    return f"r#{name}" if name in RUST_KEYWORDS else name


def parse(header_text: str):
    """(structs: [(c_name, [(field, c_type)])], enums: [(name, value)], defines, functions)."""
    text = strip_comments(header_text)
    structs = []
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} (\w+);", text, flags=re.S):
        name, body = m.group(1), m.group(2)
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            # "TYPE a, b, c" or "TYPE* a": the last token of the first item is its name
            first, *rest = [d.strip() for d in decl.split(",")]
            dm = re.fullmatch(r"(.*?[\s*])(\w+)", first)
            ctype, n0 = dm.group(1).strip(), dm.group(2)
            fields.append((n0, ctype))
            fields += [(r, ctype) for r in rest]
        structs.append((name, fields))
    enums = []
    for m in re.finditer(r"typedef enum (\w+) \{(.*?)\} (\w+);", text, flags=re.S):
        for item in m.group(2).split(","):
            item = item.strip()
            if item:
                k, v = [x.strip() for x in item.split("=")]
                enums.append((k, int(v)))
    defines = []
    for m in re.finditer(r"#define (MAMBA\w+) \(\(size_t\)(\d+) << (\d+)\)", text):
        defines.append((m.group(1), f"{m.group(2)} << {m.group(3)}"))
    body = re.sub(r"typedef (struct|enum) \w+ \{.*?\} \w+;", " ", text, flags=re.S)
    body = re.sub(r"typedef struct ihipStream_t\* mamba_stream_t;", " ", body)
    body = re.sub(r"#[^\n]*", " ", body)
    body = re.sub(r'extern "C" \{|\}', " ", body)
    functions = []
    for m in re.finditer(r"((?:const )?\w+\*?)\s+(\w+)\(([^()]*)\);", body):
        ret, name, args = m.group(1), m.group(2), " ".join(m.group(3).split())
        params = []
        if args and args != "void":
            for a in args.split(","):
                am = re.fullmatch(r"(.*?[\s*])(\w+)", a.strip())
                params.append((am.group(2), am.group(1).strip()))
        functions.append((name, ret, params))
    return structs, enums, defines, functions


def generate(header_text: str) -> str:
    structs, enums, defines, functions = parse(header_text)
    names = {s for s, _ in structs}
    out = ["// Generated from include/mamba_hip.h by gen_ffi.py: do not edit by hand.",
           "// One #[repr(C)] struct per argument struct (same fields, same order) and one",
           "// extern \"C\" declaration per entry point.",
           "#![allow(non_snake_case, non_camel_case_types, clippy::upper_case_acronyms)]",
           "",
           "use core::ffi::{c_char, c_int, c_void};",
           "",
           "/// hipStream_t (a pointer); null is the default stream.",
           "pub type MambaStream = *mut c_void;",
           ""]
    for k, v in enums:
        out.append(f"pub const {k}: c_int = {v};")
    for k, v in defines:
        out.append(f"pub const {k}: usize = {v};")
    out.append("")
    for name, fields in structs:
        out.append("#[repr(C)]")
        out.append("#[derive(Clone, Copy, Debug)]")
        out.append(f"pub struct {camel(name)} {{")
        for f, ct in fields:
            out.append(f"    pub {field_name(f)}: {rust_type(ct, names)},")
        out.append("}")
        out.append("")
        out.append(f"impl Default for {camel(name)} {{")
        out.append("    /// Every size 0, every pointer null, every stride 0.")
        out.append("    fn default() -> Self {")
        out.append("        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.")
        out.append("        unsafe { core::mem::zeroed() }")
        out.append("    }")
        out.append("}")
        out.append("")
    out.append('extern "C" {')
    for name, ret, params in functions:
        ps = ", ".join(f"{field_name(p)}: {rust_type(t, names)}" for p, t in params)
        rt = rust_type(ret, names)
        out.append(f"    pub fn {name}({ps}) -> {rt};")
    out.append("}")
    return "\n".join(out) + "\n"


def main() -> int:
    text = generate(open(HEADER).read())
    if "--check" in sys.argv[1:]:
        same = os.path.exists(OUT) and open(OUT).read() == text
        print("src/ffi.rs is up to date" if same else "src/ffi.rs is out of date: run gen_ffi.py")
        return 0 if same else 1
    with open(OUT, "w") as f:
        f.write(text)
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
