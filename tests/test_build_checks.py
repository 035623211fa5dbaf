"""The build's refusal of scratch in kernels with hand-counted memory waits,
checked on the compiler's remark text (no compile needed)."""

import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build_module():
    spec = importlib.util.spec_from_file_location("mamba_build", os.path.join(ROOT, "burn-mamba_amd", "build.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _remarks(scratch):
    out = []
    for gate in (1, 0):
        out += [f"x.hip:233:1: remark: Function Name: _ZN5mamba16mamba1_scan_tm16ILb{gate}EEEvNS_12Mamba1ParamsE",
                "x.hip:233:1: remark:     VGPRs: 122",
                f"x.hip:233:1: remark:     ScratchSize [bytes/lane]: {scratch if gate else 0}"]
    out += ["x.hip:58:1: remark: Function Name: _ZN5mamba18mamba1_scan_kernelILi16ELb1EEEvNS_12Mamba1ParamsE",
            "x.hip:58:1: remark:     ScratchSize [bytes/lane]: 64"]  # not a checked kernel
    return "\n".join(out)


def test_no_scratch_check_passes_clean_remarks():
    _build_module()._check_no_scratch("/a/mamba1.hip", _remarks(0))


def test_no_scratch_check_refuses_a_spilling_build():
    with pytest.raises(RuntimeError, match="scratch"):
        _build_module()._check_no_scratch("/a/mamba1.hip", _remarks(16))


def test_no_scratch_check_refuses_missing_remarks():
    with pytest.raises(RuntimeError, match="no resource-usage remark"):
        _build_module()._check_no_scratch("/a/mamba1.hip", "")
