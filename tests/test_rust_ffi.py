"""The Rust binding as committed source (rust/burn-mamba-hip), checked without
a Rust toolchain: src/ffi.rs is what gen_ffi.py makes of the current header;
it declares exactly the functions the library exports; and the #[repr(C)]
layout of every struct, computed from its Rust field types, equals the C
compiler's layout of the header struct (sizes and every field offset)."""

import importlib.util
import os
import re

import pytest

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


def _struct_fields(src):
    return {m.group(1): re.findall(r"pub (\w+):", m.group(2))
            for m in re.finditer(r"pub struct (\w+) \{(.*?)\n\}", src, re.S)}


def _literals(src):
    """(struct name, [field names]) of every `Name { field: value, shorthand, }`
    literal: the body split at its top-level commas."""
    out = []
    for m in re.finditer(r"\b(Mamba\w+Args) \{\n(.*?)\n\s*\};", src, re.S):
        parts, depth, cur = [], 0, ""
        for ch in m.group(2):
            depth += ch in "([{"
            depth -= ch in ")]}"
            if ch == "," and depth == 0:
                parts.append(cur)
                cur = ""
            else:
                cur += ch
        parts.append(cur)
        names = [re.match(r"\s*([A-Za-z_]\w*)", q).group(1) for q in parts if q.strip()]
        out.append((m.group(1), names))
    return out


def test_seams_fill_every_field_of_the_argument_structs():
    """src/seams.rs maps the reference's seams onto the C ABI: each argument
    struct literal names exactly the struct's fields (what rustc would check)."""
    fields = _struct_fields(open(os.path.join(CRATE, "src", "ffi.rs")).read())
    lits = _literals(open(os.path.join(CRATE, "src", "seams.rs")).read())
    assert {n for n, _ in lits} == {"MambaSsd2Args", "MambaSsd2BwdArgs", "MambaSsd3Args", "MambaSsd3DoubleArgs",
                                   "MambaSsd3BwdArgs"}
    for name, names in lits:
        assert sorted(names) == sorted(fields[name]), name
        assert len(names) == len(set(names)), name


def test_burn_arms_call_what_exists():
    """The patch's trait impls call burn_rocm functions that exist, and those
    call seams functions that exist."""
    seams = open(os.path.join(CRATE, "src", "seams.rs")).read()
    rocm = open(os.path.join(CRATE, "src", "burn_rocm.rs")).read()
    patch = open(os.path.join(CRATE, "patches", "burn-mamba-backend-rocm.patch")).read()
    seam_fns = set(re.findall(r"pub fn (\w+)\(", seams))
    rocm_fns = set(re.findall(r"pub fn (\w+)\(", rocm))
    assert set(re.findall(r"seams::(\w+)\(", rocm)) <= seam_fns
    assert set(re.findall(r"burn_mamba_hip::burn_rocm::(\w+)\(", patch)) <= rocm_fns
    for fn in ("ssd2_forward", "ssd2_backward", "ssd3_single_forward", "ssd3_double_forward"):
        assert fn in patch, fn


def test_patch_applies_to_the_reference():
    """patches/burn-mamba-backend-rocm.patch applies to the reference's own
    files (copied to a scratch directory; skipped where the reference checkout
    is absent, e.g. on the GPU box)."""
    import shutil
    import subprocess
    import tempfile
    ref = "/root/reference"
    if not os.path.isdir(ref) or shutil.which("patch") is None:
        pytest.skip("reference checkout or patch(1) not available")
    pf = os.path.join(CRATE, "patches", "burn-mamba-backend-rocm.patch")
    files = re.findall(r"^\+\+\+ b/(\S+)", open(pf).read(), re.M)
    with tempfile.TemporaryDirectory() as tmp:
        for f in files:
            os.makedirs(os.path.dirname(os.path.join(tmp, f)) or tmp, exist_ok=True)
            shutil.copy(os.path.join(ref, f), os.path.join(tmp, f))
        r = subprocess.run(["patch", "-p1", "--dry-run", "-i", pf], cwd=tmp, capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr
