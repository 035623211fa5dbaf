"""Mamba-3 single-pass SSD: mamba_ssd3_fwd (C ABI) vs the CPU oracle (serial
K1-K5 restatement of the reference, pinned by the trapezoid recurrence and the
lambda = 1 -> Mamba-2 reduction).  f32 at rtol 1e-4, bf16 I/O at rtol 2e-2 /
atol 1e-2; final states in every case."""

import numpy as np
import pytest

from inputs import bf16_round, ssd3_inputs

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=2e-5)
BF16_TOL = dict(rtol=2e-2, atol=1e-2)


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


CASES = [
    # (b, l, m, h, p, n, chunk, io)
    (2, 64, 1, 3, 16, 8, 16, "f32"),     # SISO
    (1, 50, 2, 2, 8, 12, 8, "f32"),      # ragged seqlen
    (2, 40, 4, 2, 16, 16, 8, "f32"),     # MIMO 4
    (1, 37, 4, 2, 64, 32, 16, "f32"),    # headdim 64, ragged
    (1, 96, 4, 2, 64, 128, 32, "bf16"),  # config-4 head shape, bf16 I/O
]


@pytest.mark.parametrize("case", CASES)
def test_ssd3_matches_oracle(case):
    import torch
    import mamba_hip
    import oracle
    b, l, m, h, p, n, q, io = case
    d = ssd3_inputs(sum(case[:6]), b, l, m, h, p, n)
    dt = torch.float32 if io == "f32" else torch.bfloat16
    v, B, C = (d[k] if io == "f32" else bf16_round(d[k]) for k in ("v", "B", "C"))
    y, hT = mamba_hip.ssd3_fwd(_t(v, dt), _t(d["da"]), _t(B, dt), _t(C, dt), _t(d["gamma"]), _t(d["scale"]),
                               _t(d["h0"]), chunk_len=q)
    torch.cuda.synchronize()
    yr, hr = oracle.ssd3(v, d["da"], B, C, d["gamma"], d["scale"], d["h0"], chunk=q)
    tol = F32_TOL if io == "f32" else BF16_TOL
    np.testing.assert_allclose(y.float().cpu().numpy(), yr, **tol)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **F32_TOL if io == "f32" else dict(rtol=1e-3, atol=1e-3))


def test_ssd3_shared_groups_and_no_initial_state():
    """ngroups < nheads (B/C shared by heads) and a NULL initial state."""
    import torch
    import mamba_hip
    import oracle
    b, l, m, h, p, n = 1, 30, 2, 4, 8, 8
    d = ssd3_inputs(5, b, l, m, h, p, n)
    Bg, Cg = d["B"][:, :, :, :2], d["C"][:, :, :, :2]  # two groups
    y, hT = mamba_hip.ssd3_fwd(_t(d["v"]), _t(d["da"]), _t(Bg), _t(Cg), _t(d["gamma"]), _t(d["scale"]), None,
                               chunk_len=8)
    torch.cuda.synchronize()
    Bh, Ch = np.repeat(Bg, 2, axis=3), np.repeat(Cg, 2, axis=3)
    yr, hr = oracle.ssd3(d["v"], d["da"], Bh, Ch, d["gamma"], d["scale"], None, chunk=8)
    np.testing.assert_allclose(y.cpu().numpy(), yr, **F32_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **F32_TOL)


def test_ssd3_chunk_independence_and_split():
    """y does not depend on chunk_len; two calls carrying the state equal one."""
    import torch
    import mamba_hip
    b, l, m, h, p, n = 1, 48, 4, 2, 16, 16
    d = ssd3_inputs(9, b, l, m, h, p, n)
    args = [_t(d[k]) for k in ("v", "da", "B", "C", "gamma", "scale")]
    y1, h1 = mamba_hip.ssd3_fwd(*args, _t(d["h0"]), chunk_len=8)
    y2, h2 = mamba_hip.ssd3_fwd(*args, _t(d["h0"]), chunk_len=16)
    cut = 24
    part = lambda a, s: a[:, s].contiguous()  # noqa: E731
    ya, ha = mamba_hip.ssd3_fwd(*[part(a, slice(0, cut)) for a in args], _t(d["h0"]), chunk_len=8)
    yb, hb = mamba_hip.ssd3_fwd(*[part(a, slice(cut, l)) for a in args], ha, chunk_len=8)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y1.cpu().numpy(), y2.cpu().numpy(), **F32_TOL)
    np.testing.assert_allclose(h1.cpu().numpy(), h2.cpu().numpy(), **F32_TOL)
    np.testing.assert_allclose(torch.cat([ya, yb], 1).cpu().numpy(), y1.cpu().numpy(), **F32_TOL)
    np.testing.assert_allclose(hb.cpu().numpy(), h1.cpu().numpy(), **F32_TOL)


def test_mamba3_single_ssd_input_run():
    """The reference bundle: init_state_hpr adds to the initial state."""
    import torch
    import mamba_hip
    import oracle
    b, l, m, h, p, n = 2, 20, 2, 2, 8, 8
    d = ssd3_inputs(11, b, l, m, h, p, n)
    hpr = (0.05 * np.random.default_rng(0).standard_normal((h, p, n))).astype(np.float32)
    inp = mamba_hip.Mamba3SingleSsdInput(_t(d["v"]), _t(d["B"]), _t(d["C"]), _t(d["da"]), _t(d["gamma"]),
                                         _t(d["scale"]), _t(d["h0"]), _t(hpr))
    y, hT = inp.run(chunk_len=8)
    torch.cuda.synchronize()
    yr, hr = oracle.ssd3(d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], d["h0"] + hpr[None], chunk=8)
    np.testing.assert_allclose(y.cpu().numpy(), yr, **F32_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **F32_TOL)


# ---------------------------------------------------------------- MFMA path --
# bf16 I/O, headdim 64, dstate 128, MIMO rank dividing 32: the single-kernel
# MFMA path (128 fused positions per chunk, state held on chip).
MFMA_CASES = [
    # (b, l, m, h, g, p, n, with_h0)
    (2, 200, 4, 4, 4, 64, 128, True),   # ragged: 800 fused positions = 6.25 chunks
    (1, 300, 1, 2, 2, 64, 128, True),   # SISO
    (1, 130, 2, 2, 2, 64, 128, True),   # MIMO 2, ragged
    (1, 70, 8, 2, 2, 64, 128, True),    # MIMO 8
    (1, 9, 32, 2, 2, 64, 128, True),    # MIMO 32: one step per 32-row tile
    (1, 100, 4, 4, 2, 64, 128, False),  # shared groups, NULL initial state
    (1, 3, 4, 1, 1, 64, 128, True),     # shorter than one tile
]


def _mfma_inputs(case):
    b, l, m, h, g, p, n, with_h0 = case
    d = ssd3_inputs(sum(case[:7]), b, l, m, h, p, n)
    rep = h // g
    B, C = bf16_round(d["B"][:, :, :, ::rep]), bf16_round(d["C"][:, :, :, ::rep])
    return d, bf16_round(d["v"]), B, C, (d["h0"] if with_h0 else None), rep


@pytest.mark.parametrize("case", MFMA_CASES)
def test_ssd3_mfma_matches_oracle(case):
    import torch
    import mamba_hip
    import oracle
    d, v, B, C, h0, rep = _mfma_inputs(case)
    bf = torch.bfloat16
    args = (_t(v, bf), _t(d["da"]), _t(B, bf), _t(C, bf), _t(d["gamma"]), _t(d["scale"]))
    assert mamba_hip.ssd3_fast_path(*args, chunk_len=32)
    y, hT = mamba_hip.ssd3_fwd(*args, None if h0 is None else _t(h0), chunk_len=32)
    torch.cuda.synchronize()
    Bh, Ch = np.repeat(B, rep, axis=3), np.repeat(C, rep, axis=3)
    yr, hr = oracle.ssd3(v, d["da"], Bh, Ch, d["gamma"], d["scale"], h0, chunk=32)
    np.testing.assert_allclose(y.float().cpu().numpy(), yr, **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, rtol=1e-2, atol=5e-3)


def test_ssd3_fast_path_predicate():
    import torch
    import mamba_hip
    d = ssd3_inputs(1, 1, 16, 4, 2, 64, 128)
    bf = torch.bfloat16
    ok = lambda v, B, C: mamba_hip.ssd3_fast_path(v, _t(d["da"]), B, C, _t(d["gamma"]), _t(d["scale"]))  # noqa: E731
    assert ok(_t(d["v"], bf), _t(d["B"], bf), _t(d["C"], bf))
    assert not ok(_t(d["v"]), _t(d["B"]), _t(d["C"]))  # f32 I/O
    d3 = ssd3_inputs(1, 1, 16, 3, 2, 64, 128)
    assert not mamba_hip.ssd3_fast_path(_t(d3["v"], bf), _t(d3["da"]), _t(d3["B"], bf), _t(d3["C"], bf),
                                        _t(d3["gamma"]), _t(d3["scale"]))  # MIMO 3
    d4 = ssd3_inputs(1, 1, 16, 4, 2, 32, 128)
    assert not mamba_hip.ssd3_fast_path(_t(d4["v"], bf), _t(d4["da"]), _t(d4["B"], bf), _t(d4["C"], bf),
                                        _t(d4["gamma"]), _t(d4["scale"]))  # headdim 32


def test_ssd3_mfma_matches_generic_strided():
    """Fast path vs the generic kernels on the same bf16 inputs, with v and y
    as headdim slices of wider tensors (non-default head/position strides)."""
    import torch
    import mamba_hip
    b, l, m, h, p, n = 2, 512, 4, 4, 64, 128
    d = ssd3_inputs(21, b, l, m, h, p, n)
    bf = torch.bfloat16
    wide = torch.zeros((b, l, m, h, 2 * p), dtype=bf, device="cuda")
    wide[..., p:] = _t(d["v"], bf)
    v = wide[..., p:]
    yw = torch.full((b, l, m, h, 2 * p), 7.0, dtype=bf, device="cuda")
    rest = (_t(d["da"]), _t(d["B"], bf), _t(d["C"], bf), _t(d["gamma"]), _t(d["scale"]))
    assert mamba_hip.ssd3_fast_path(v, *rest)
    y, hT = mamba_hip.ssd3_fwd(v, *rest, _t(d["h0"]), chunk_len=32, y=yw[..., :p])
    yg, hg = mamba_hip.ssd3_fwd(v.contiguous(), *rest, _t(d["h0"]), chunk_len=32, generic=True)
    torch.cuda.synchronize()
    assert bool((yw[..., p:] == 7.0).all()), "write outside the y slice"
    np.testing.assert_allclose(y.float().cpu().numpy(), yg.float().cpu().numpy(), **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hg.cpu().numpy(), rtol=1e-2, atol=5e-3)


def test_ssd3_mfma_split_carries_state():
    """Two fast-path calls chained through the final state equal one call."""
    import torch
    import mamba_hip
    b, l, m, h, p, n = 1, 256, 4, 2, 64, 128
    d = ssd3_inputs(23, b, l, m, h, p, n)
    bf = torch.bfloat16
    args = [_t(d["v"], bf), _t(d["da"]), _t(d["B"], bf), _t(d["C"], bf), _t(d["gamma"]), _t(d["scale"])]
    y1, h1 = mamba_hip.ssd3_fwd(*args, _t(d["h0"]))
    cut = 96  # 384 fused positions: ends mid-chunk
    part = lambda a, s: a[:, s].contiguous()  # noqa: E731
    ya, ha = mamba_hip.ssd3_fwd(*[part(a, slice(0, cut)) for a in args], _t(d["h0"]))
    yb, hb = mamba_hip.ssd3_fwd(*[part(a, slice(cut, l)) for a in args], ha)
    torch.cuda.synchronize()
    np.testing.assert_allclose(torch.cat([ya, yb], 1).float().cpu().numpy(), y1.float().cpu().numpy(), **BF16_TOL)
    np.testing.assert_allclose(hb.cpu().numpy(), h1.cpu().numpy(), rtol=1e-2, atol=5e-3)
