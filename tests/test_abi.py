"""C-ABI checks that need no GPU: the library loads, exports exactly the
functions include/mamba_hip.h declares, and the ctypes struct mirrors have the
C layout (sizes and field offsets compiled by gcc from the header)."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mamba_hip.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(mamba\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_header_declares_what_binding_binds():
    import mamba_hip
    assert _declared_functions() == mamba_hip.exported_symbols()


def test_library_loads_and_exports_every_symbol():
    import mamba_hip
    L = mamba_hip.lib()
    for name in _declared_functions():
        assert hasattr(L, name), name
    assert L.mamba_version().decode().startswith("mamba_hip")


def _c_layout(struct_name, fields):
    body = "\n".join(f'printf("%zu\\n", offsetof({struct_name}, {f}));' for f in fields)
    prog = f"""#include <stdio.h>
#include <stddef.h>
#include "mamba_hip.h"
int main(void) {{ printf("%zu\\n", sizeof({struct_name})); {body} return 0; }}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "p.c")
        exe = os.path.join(d, "p")
        open(c, "w").write(prog)
        subprocess.run(["gcc", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    return [int(v) for v in out]


@pytest.mark.parametrize("cls_name,c_name", [("Ssd2Args", "mamba_ssd2_args"), ("Ssd3Args", "mamba_ssd3_args"),
                                             ("Ssd3DoubleArgs", "mamba_ssd3_double_args"),
                                             ("Mamba1ScanArgs", "mamba1_scan_args"),
                                             ("Mamba1StepArgs", "mamba1_step_args"),
                                             ("Conv1dStepArgs", "mamba_conv1d_step_args"),
                                             ("Mamba2StepArgs", "mamba2_step_args"),
                                             ("Mamba3StepArgs", "mamba3_step_args"),
                                             ("Mamba3PrepArgs", "mamba3_prep_args"),
                                             ("Mamba3FinishArgs", "mamba3_finish_args"),
                                             ("Mamba3FusedArgs", "mamba3_fused_args"),
                                             ("Ssd2BwdArgs", "mamba_ssd2_bwd_args"),
                                             ("Ssd3BwdArgs", "mamba_ssd3_bwd_args"),
                                             ("Mamba3DoubleInputsArgs", "mamba3_double_inputs_args"),
                                             ("LinearArgs", "mamba_linear_args"),
                                             ("Mamba2LayerArgs", "mamba2_layer_args"),
                                             ("RmsNormArgs", "mamba_rmsnorm_args"),
                                             ("Mamba2ConvArgs", "mamba2_conv_args"),
                                             ("Mamba2GatedNormArgs", "mamba2_gated_norm_args")])
def test_struct_layouts_match_header(cls_name, c_name):
    from mamba_hip import _lib
    cls = getattr(_lib, cls_name)
    fields = [f[0] for f in cls._fields_]
    got = _c_layout(c_name, fields)
    assert got[0] == ctypes.sizeof(cls)
    assert got[1:] == [getattr(cls, f).offset for f in fields]


def test_invalid_args_need_no_gpu():
    """Host-side validation rejects bad shapes before any HIP call."""
    from mamba_hip import _lib
    a = _lib.Ssd2Args()
    a.batch, a.seqlen, a.nheads, a.headdim, a.ngroups, a.dstate, a.chunk_len = 1, 8, 3, 4, 2, 4, 4
    rc = _lib.lib().mamba_ssd2_fwd(ctypes.byref(a), None, 0, None)
    assert rc == 1  # MAMBA_ERR_INVALID_ARG
    assert b"ngroups" in _lib.lib().mamba_last_error()


def test_step_validation_needs_no_gpu():
    """mamba2_step_ssm rejects bad groups and a short workspace before any HIP call."""
    from mamba_hip import _lib
    L = _lib.lib()
    a = _lib.Mamba2StepArgs()
    a.batch, a.nheads, a.headdim, a.ngroups, a.dstate, a.conv_kernel = 2, 3, 64, 2, 128, 4
    assert L.mamba2_step_ssm(ctypes.byref(a), None, 0, None) == 1
    assert b"ngroups" in L.mamba_last_error()
    a.nheads = 4
    for name in ("zxbcdt", "conv_state", "conv_w", "A", "norm_w", "ssm_state", "out"):
        setattr(a, name, 4096)  # never dereferenced: validation fails first
    a.zxbcdt_sb = 4 * 64 + 4 * 64 + 2 * 2 * 128 + 4
    a.out_sb = 4 * 64
    need = L.mamba2_step_workspace_size(ctypes.byref(a))
    assert need >= 2 * 4 * 64 * 4
    assert L.mamba2_step_ssm(ctypes.byref(a), ctypes.c_void_p(4096), need - 1, None) == 3  # WORKSPACE
    assert b"workspace" in L.mamba_last_error()
    r = _lib.RmsNormArgs()
    r.rows, r.cols = 2, 8
    assert L.mamba_rmsnorm(ctypes.byref(r), None) == 1


def test_fused_predicate_needs_no_gpu():
    """mamba3_ssd_fused_supported validates and classifies host-side: 1 at the
    config-4 shape, 0 outside the fused kernel's shapes / layouts, -1 for
    invalid arguments (no pointer is dereferenced)."""
    from mamba_hip import _lib
    L = _lib.lib()
    a = _lib.Mamba3FusedArgs()
    p = a.prep
    p.batch, p.seqlen, p.nheads, p.headdim, p.ngroups, p.dstate, p.mimo, p.rope_dim = 4, 8192, 32, 64, 1, 128, 4, 128
    p.proj_dtype = p.io_dtype = 1  # MAMBA_BF16
    p.proj_sl = 2 * 32 * 64 + 2 * 4 * 128 + 3 * 32 + 64
    p.proj_sb = 8192 * p.proj_sl
    ptrs = ("proj", "ssm_state", "k_state", "v_state", "angle", "angle_out", "dt_bias", "b_norm_w", "c_norm_w",
            "b_bias", "c_bias", "mimo_x", "initial_state")
    for i, name in enumerate(ptrs):
        setattr(p, name, 4096 * (i + 1))  # never dereferenced
    a.y, a.final_state = 4096 * 20, 4096 * 21
    assert L.mamba3_ssd_fused_supported(ctypes.byref(a)) == 1
    p.mimo = 1  # SISO (its in_proj row is shorter than proj_sl: allowed)
    assert L.mamba3_ssd_fused_supported(ctypes.byref(a)) == 1
    p.mimo = 4
    for field, bad in (("headdim", 32), ("proj_dtype", 0)):
        old = getattr(p, field)
        setattr(p, field, bad)
        assert L.mamba3_ssd_fused_supported(ctypes.byref(a)) == 0, field
        setattr(p, field, old)
    p.proj_sl += 4  # rows no longer 16-byte aligned
    p.proj_sb = 8192 * p.proj_sl
    assert L.mamba3_ssd_fused_supported(ctypes.byref(a)) == 0
    a.y = None
    assert L.mamba3_ssd_fused_supported(ctypes.byref(a)) == -1
    assert L.mamba3_ssd_fused_fwd(ctypes.byref(a), None) == 1
    assert b"y and final_state" in L.mamba_last_error()


def test_missing_library_raises_no_fallback():
    """The product path has no CPU fallback: with libmamba_hip.so absent, the
    first library call raises MambaHipError (checked in a fresh interpreter,
    so the library already loaded by this process is not reused)."""
    import sys
    code = (
        "import sys; sys.path[:0] = [%r]\n"
        "from mamba_hip import _lib\n"
        "_lib.LIB_PATH = '/nonexistent/libmamba_hip.so'\n"
        "try:\n"
        "    _lib.lib()\n"
        "except _lib.MambaHipError as e:\n"
        "    print('raised', e)\n"
        "    sys.exit(0)\n"
        "sys.exit(3)\n" % os.path.join(ROOT, "burn-mamba_amd"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "raised" in r.stdout, r.stdout + r.stderr


def test_batch_parts_need_no_gpu():
    """The batch-split decode schedule: batch_parts gives ceil(b / 32) row parts
    for 34 to 256 rows, at least 2 and at most the stack's cap; Mamba2Stack
    caps at two (halves) and applies to a fused stack only, Mamba3Stack at
    four; both can be switched off."""
    import mamba_hip

    bs = (1, 16, 32, 33, 34, 35, 36, 48, 64, 65, 66, 96, 97, 100, 128, 255, 256, 258)
    assert [mamba_hip.batch_parts(b, 4) for b in bs] == [1, 1, 1, 1, 2, 2, 2, 2, 2, 3, 3, 3, 4, 4, 4, 4, 4, 1]
    assert [mamba_hip.batch_parts(b, 2) for b in bs] == [1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 1]

    def stack(fused, split_batch):  # the predicate reads only these two flags; no layers are built
        s = object.__new__(mamba_hip.Mamba2Stack)
        s.fused, s.split_batch = fused, split_batch
        return s

    s = stack(True, True)
    assert [b for b in bs if s.splits(b)] == [34, 35, 36, 48, 64, 65, 66, 96, 97, 100, 128, 255, 256]
    assert all(s.parts(b) == 2 for b in bs if s.splits(b))
    assert not stack(True, False).splits(64)
    assert not stack(False, True).splits(64)
    m3 = object.__new__(mamba_hip.Mamba3Stack)
    m3.split_batch = True
    assert [m3.parts(b) for b in (33, 34, 48, 64, 96, 100, 128, 256)] == [1, 2, 2, 2, 3, 4, 4, 4]
    m3.split_batch = False
    assert m3.parts(100) == 1
