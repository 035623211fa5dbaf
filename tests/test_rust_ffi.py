"""The Rust binding as committed source (rust/burn-mamba-hip), checked without
a Rust toolchain: src/ffi.rs is what gen_ffi.py makes of the current header;
it declares exactly the functions the library exports; and the #[repr(C)]
layout of every struct, computed from its Rust field types, equals the C
compiler's layout of the header struct (sizes and every field offset)."""

import importlib.util
import os
import re

from test_abi import _c_layout, _declared_functions

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "rust", "burn-mamba-hip")


def _gen():
    spec = importlib.util.spec_from_file_location("gen_ffi", os.path.join(CRATE, "gen_ffi.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_ffi_rs_matches_the_header():
    g = _gen()
    want = g.generate(open(os.path.join(ROOT, "include", "mamba_hip.h")).read())
    assert open(os.path.join(CRATE, "src", "ffi.rs")).read() == want, "run rust/burn-mamba-hip/gen_ffi.py"


def test_ffi_rs_declares_every_entry_point():
    ffi = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    declared = sorted(re.findall(r"pub fn (mamba\w+)\(", ffi))
    assert declared == _declared_functions()


_SIZE = {"i32": 4, "u32": 4, "f32": 4, "c_int": 4, "i64": 8, "f64": 8, "usize": 8}


def _rust_layout(structs, name):
    """(size, align, [offsets]) of a #[repr(C)] struct from its Rust field types."""
    off, align, offs = 0, 1, []
    for _, t in structs[name]:
        if t.startswith("*") or t == "MambaStream":
            s = a = 8
        elif t in _SIZE:
            s = a = _SIZE[t]
        else:
            s, a, _ = _rust_layout(structs, t)
        off = (off + a - 1) // a * a
        offs.append(off)
        off += s
        align = max(align, a)
    return (off + align - 1) // align * align, align, offs


def test_repr_c_layouts_equal_the_c_layouts():
    g = _gen()
    header = open(os.path.join(ROOT, "include", "mamba_hip.h")).read()
    cstructs, _, _, _ = g.parse(header)
    names = {n for n, _ in cstructs}
    rs = {g.camel(n): [(f, g.rust_type(t, names)) for f, t in fields] for n, fields in cstructs}
    for cname, fields in cstructs:
        size, _, offs = _rust_layout(rs, g.camel(cname))
        got = _c_layout(cname, [f for f, _ in fields])
        assert got[0] == size, cname
        assert got[1:] == offs, cname


def test_library_version_matches_the_crate():
    import mamba_hip
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    want = re.search(r'^version = "([^"]+)"', cargo, re.M).group(1)
    assert mamba_hip.lib().mamba_version().decode().split()[1] == want
