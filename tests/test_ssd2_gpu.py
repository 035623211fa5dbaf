"""Mamba-2 SSD: libmamba_hip.so (through the C ABI) vs the CPU oracle.

Tolerances: f32 I/O rtol 1e-4 (with a small atol
for values near zero); bf16 inputs with f32 accumulation: rtol 2e-2 and
atol 1e-2 on y; final states are compared in every case.  The oracle is fed
exactly the bf16-rounded inputs the GPU sees.
"""

import numpy as np
import pytest

from inputs import bf16_round, ssd2_inputs, ssd2_test_inputs

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=1e-5)
BF16_TOL = dict(rtol=2e-2, atol=1e-2)


def _run_gpu(inp, chunk, dtype, generic=False, dt_layout="blh", per_head=False):
    import torch
    import mamba_hip
    dev = torch.device("cuda:0")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = torch.from_numpy(inp["x"]).to(dev, tdt)
    Bm = torch.from_numpy(inp["B"]).to(dev, tdt)
    Cm = torch.from_numpy(inp["C"]).to(dev, tdt)
    if per_head:
        h = x.shape[2]
        g = Bm.shape[2]
        Bm = Bm.repeat_interleave(h // g, dim=2)
        Cm = Cm.repeat_interleave(h // g, dim=2)
    dt = torch.from_numpy(inp["dt"]).to(dev)
    if dt_layout == "bhl":  # the reference seam's dt_bhnl layout, as a strided view
        dt = dt.permute(0, 2, 1).contiguous().permute(0, 2, 1)
    A = torch.from_numpy(inp["A"]).to(dev)
    D = None if inp["D"] is None else torch.from_numpy(inp["D"]).to(dev)
    h0 = None if inp["h0"] is None else torch.from_numpy(inp["h0"]).to(dev)
    y, hT = mamba_hip.ssd2_fwd(x, dt, A, Bm, Cm, D, h0, chunk_len=chunk, generic=generic)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), hT.cpu().numpy()


def _oracle(inp, chunk, dtype):
    import oracle
    x, B, C = inp["x"], inp["B"], inp["C"]
    if dtype == "bf16":
        x, B, C = bf16_round(x), bf16_round(B), bf16_round(C)
    return oracle.ssd2(x, inp["dt"], inp["A"], B, C, inp["D"], inp["h0"], chunk=chunk)


CASES = [
    # (b, l, h, p, g, n, chunk)
    (2, 512, 8, 64, 1, 64, 64),     # config 0
    (2, 37, 4, 8, 2, 8, 8),         # ragged tail, GQA 2 groups
    (1, 1, 2, 16, 1, 16, 64),       # single token
    (2, 300, 4, 64, 1, 128, 96),    # reference optimal chunk (96) for r=128,p=64, ragged
    (1, 256, 4, 32, 4, 32, 256),    # per-group == per-head, one chunk
    (3, 130, 6, 16, 3, 24, 32),     # odd dims
]


@pytest.mark.parametrize("generic", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_ssd2_f32(case, generic):
    b, l, h, p, g, n, q = case
    inp = ssd2_inputs(seed=hash(case) % 1000, b=b, l=l, h=h, p=p, g=g, n=n, h0=True)
    y, hT = _run_gpu(inp, q, "f32", generic=generic)
    yr, hr = _oracle(inp, q, "f32")
    np.testing.assert_allclose(y, yr, **F32_TOL)
    np.testing.assert_allclose(hT, hr, **F32_TOL)


@pytest.mark.parametrize("generic", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_ssd2_bf16(case, generic):
    b, l, h, p, g, n, q = case
    inp = ssd2_inputs(seed=7 + hash(case) % 1000, b=b, l=l, h=h, p=p, g=g, n=n, h0=True)
    y, hT = _run_gpu(inp, q, "bf16", generic=generic)
    yr, hr = _oracle(inp, q, "bf16")
    np.testing.assert_allclose(y, yr, **BF16_TOL)
    np.testing.assert_allclose(hT, hr, **BF16_TOL)


def test_ssd2_reference_test_distribution():
    """The reference's own agreement-test shapes and distributions
    (src/mamba2/ssd/ssd_path/tests.rs:33-67, 184-336)."""
    for (b, n_, l_, h, p, r) in [(2, 3, 4, 2, 8, 8), (2, 3, 4, 4, 8, 8), (2, 1, 4, 2, 8, 8)]:
        inp = ssd2_test_inputs(seed=11, b=b, l=n_ * l_, h=h, p=p, g=h, n=r)
        y, hT = _run_gpu(inp, l_, "f32")
        yr, hr = _oracle(inp, l_, "f32")
        np.testing.assert_allclose(y, yr, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(hT, hr, rtol=1e-4, atol=1e-4)


def test_ssd2_seam_layouts():
    """The Mamba2BackendExt seam passes dt as [b,h,n,l] and per-head B/C
    (serial_recalculated.rs:48; mamba2.rs:733-734): same result."""
    inp = ssd2_inputs(seed=3, b=2, l=256, h=8, p=64, g=1, n=64, h0=True)
    y0, h0 = _run_gpu(inp, 64, "f32")
    y1, h1 = _run_gpu(inp, 64, "f32", dt_layout="bhl", per_head=True)
    np.testing.assert_allclose(y1, y0, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(h1, h0, rtol=1e-5, atol=1e-6)


def test_ssd2_golden_fixture():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "ssd2_cfg0_small.npz")
    f = np.load(path)
    inp = dict(x=f["x"], dt=f["dt"], A=f["A"], B=f["B"], C=f["C"], D=f["D"], h0=f["h0"])
    y, hT = _run_gpu(inp, int(f["chunk"]), "f32")
    np.testing.assert_allclose(y, f["y"], **F32_TOL)
    np.testing.assert_allclose(hT, f["final_state"], **F32_TOL)


def test_ssd2_invalid_args_rejected():
    import torch
    import mamba_hip
    dev = torch.device("cuda:0")
    x = torch.zeros(1, 8, 3, 4, device=dev)
    dt = torch.zeros(1, 8, 3, device=dev)
    A = torch.zeros(3, device=dev)
    Bm = torch.zeros(1, 8, 2, 4, device=dev)  # 3 heads not a multiple of 2 groups
    with pytest.raises(mamba_hip.MambaHipError, match="ngroups"):
        mamba_hip.ssd2_fwd(x, dt, A, Bm, Bm, chunk_len=4)


# ------------------------------------------------- MFMA fast path (bf16) ----

FAST_CASES = [
    # (b, l, h, p, g, n, chunk)
    (1, 1024, 8, 64, 1, 128, 256),   # config-1 head shape, reduced batch/length
    (2, 1000, 4, 64, 2, 128, 256),   # ragged tail, 2 groups
    (2, 333, 6, 64, 3, 64, 64),      # dstate 64, ragged
    (1, 77, 2, 64, 1, 128, 32),      # smallest chunk
    (1, 512, 4, 64, 1, 64, 160),     # chunk 160 (the kernel chunks at 128)
    (3, 256, 80, 64, 1, 128, 256),   # all 80 heads of config 1
    (2, 700, 10, 64, 1, 128, 96),    # 10 heads: sets of 5, eight chunks of 96, ragged
    (1, 450, 20, 64, 2, 64, 128),    # dstate 64 with sets of 5 per group
]


def _hpw_ok(h, g, hpw):
    return (h // g) % hpw == 0


def _to_dev(inp, dtype="bf16"):
    import torch
    dev = torch.device("cuda:0")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    return dict(
        x=torch.from_numpy(inp["x"]).to(dev, tdt), B=torch.from_numpy(inp["B"]).to(dev, tdt),
        C=torch.from_numpy(inp["C"]).to(dev, tdt), dt=torch.from_numpy(inp["dt"]).to(dev),
        A=torch.from_numpy(inp["A"]).to(dev),
        D=None if inp["D"] is None else torch.from_numpy(inp["D"]).to(dev),
        h0=None if inp["h0"] is None else torch.from_numpy(inp["h0"]).to(dev))


@pytest.mark.parametrize("hpw", [1, 2, 4, 5])
@pytest.mark.parametrize("case", FAST_CASES)
def test_ssd2_mfma_bf16(case, hpw, monkeypatch):
    """The MFMA path at every head-set size it can run a shape with
    (MAMBA_SSD2_HPW forces the choice)."""
    import torch
    import mamba_hip
    b, l, h, p, g, n, q = case
    if not _hpw_ok(h, g, hpw):
        pytest.skip(f"{h // g} heads per group do not split into sets of {hpw}")
    monkeypatch.setenv("MAMBA_SSD2_HPW", str(hpw))
    inp = ssd2_inputs(seed=100 + sum(case), b=b, l=l, h=h, p=p, g=g, n=n, h0=True)
    t = _to_dev(inp)
    assert mamba_hip.ssd2_fast_path(t["x"], t["dt"], t["A"], t["B"], t["C"], chunk_len=q)
    y, hT = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["h0"], chunk_len=q)
    torch.cuda.synchronize()
    yr, hr = _oracle(inp, q, "bf16")
    np.testing.assert_allclose(y.float().cpu().numpy(), yr, **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **BF16_TOL)


def test_ssd2_mfma_zero_state_and_init_hpr():
    """No initial state (the config-1 case) and the learnable init_state_hpr
    (added to h0 as minimal.rs:316-328 does) on the fast path."""
    import torch
    import mamba_hip
    import oracle
    inp = ssd2_inputs(seed=5, b=2, l=600, h=4, p=64, g=1, n=128, h0=False)
    t = _to_dev(inp)
    y, hT = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], None, chunk_len=256)
    torch.cuda.synchronize()
    yr, hr = _oracle(inp, 256, "bf16")
    np.testing.assert_allclose(y.float().cpu().numpy(), yr, **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **BF16_TOL)
    init = (0.1 * np.random.default_rng(1).standard_normal((4, 64, 128))).astype(np.float32)
    y2, h2 = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], None,
                                torch.from_numpy(init).cuda(), chunk_len=256)
    torch.cuda.synchronize()
    xr, Br, Cr = bf16_round(inp["x"]), bf16_round(inp["B"]), bf16_round(inp["C"])
    yr2, hr2 = oracle.ssd2(xr, inp["dt"], inp["A"], Br, Cr, inp["D"], None, init, chunk=256)
    np.testing.assert_allclose(y2.float().cpu().numpy(), yr2, **BF16_TOL)
    np.testing.assert_allclose(h2.cpu().numpy(), hr2, **BF16_TOL)


def test_ssd2_mfma_matches_generic_closely():
    """Fast path vs the f32 SIMT path on identical bf16 inputs: differences
    come only from the bf16 rounding of the MFMA operands."""
    import torch
    import mamba_hip
    inp = ssd2_inputs(seed=9, b=1, l=768, h=8, p=64, g=1, n=128, h0=True)
    t = _to_dev(inp)
    yf, hf = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["h0"], chunk_len=256)
    yg, hg = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["h0"], chunk_len=256,
                                generic=True)
    torch.cuda.synchronize()
    np.testing.assert_allclose(yf.float().cpu().numpy(), yg.float().cpu().numpy(), **BF16_TOL)
    np.testing.assert_allclose(hf.cpu().numpy(), hg.cpu().numpy(), **BF16_TOL)


@pytest.mark.parametrize("dt_range", [(0.02, 1.5), (0.5, 4.0)])
def test_ssd2_mfma_steep_blocks(dt_range):
    """Strong decay.  A 32-position block whose total decay exp(sum dt A) is
    below 2^-64 takes the exact per-element diagonal path; the others take the
    factored one.  Both kinds occur in these inputs (checked below) and both
    must match the oracle, outputs and final states."""
    import torch
    import mamba_hip
    b, l, h, g, q = 2, 700, 8, 2, 256
    inp = ssd2_inputs(seed=31, b=b, l=l, h=h, p=64, g=g, n=128, h0=True, dt_range=dt_range)
    lp = -(-l // 32) * 32
    da2 = np.zeros((b, lp, h))
    da2[:, :l] = inp["dt"] * inp["A"][None, None, :] * np.log2(np.e)
    span = -da2.reshape(b, lp // 32, 32, h).sum(axis=2)
    assert (span > 64).any()
    if dt_range[0] < 0.1:
        assert (span <= 64).any()
    t = _to_dev(inp)
    y, hT = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["h0"], chunk_len=q)
    torch.cuda.synchronize()
    yr, hr = _oracle(inp, q, "bf16")
    np.testing.assert_allclose(y.float().cpu().numpy(), yr, **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **BF16_TOL)


def _assert_close_rows(got, want, rtol, atol, what):
    """assert_allclose over the leading axis, one slice at a time (the
    full-size arrays are hundreds of MB)."""
    for i in range(got.shape[0]):
        np.testing.assert_allclose(got[i], want[i], rtol=rtol, atol=atol, err_msg=f"{what}[{i}]")


def test_ssd2_config1_full_size():
    """BASELINE.json configs[1] at its full size (8 x 4096 tokens, 80 heads,
    headdim 64, dstate 128, one group, chunk 256, bf16 x/B/C/y): the benched
    MFMA path (16-chunk state carry, XCD-remapped workgroups) against the f32
    serial oracle on the same bf16-rounded inputs; y and the final state at
    north_star's bf16 bars."""
    import torch
    import mamba_hip
    import oracle
    b, l, h, p, g, n, q = 8, 4096, 80, 64, 1, 128, 256
    print(f"ssd2 config 1 full size {b}x{l}x{h}", flush=True)
    inp = ssd2_inputs(seed=2024, b=b, l=l, h=h, p=p, g=g, n=n, h0=False)
    t = _to_dev(inp)
    assert mamba_hip.ssd2_fast_path(t["x"], t["dt"], t["A"], t["B"], t["C"], chunk_len=q)
    y, hT = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], None, chunk_len=q)
    torch.cuda.synchronize()
    y = y.float().cpu().numpy()
    hT = hT.cpu().numpy()
    del t
    for k in ("x", "B", "C"):
        inp[k] = bf16_round(inp[k])
    yr, hr = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], None, chunk=q,
                         form="serial", prec=32)
    _assert_close_rows(y, yr, what="y", **BF16_TOL)
    _assert_close_rows(hT, hr, what="final_state", **BF16_TOL)


def test_mamba2_ssd_input_run_chunked():
    """Mamba2SsdInput.run on the reference's 5-d chunked tensors
    (ssd_path.rs:58-87, 149-155): x [b, n, l, h, p], dt [b, n, l, h], per-head
    B/C [b, n, l, h, r] as the reference's GQA expand leaves them
    (mamba2.rs:733-734), and a learnable init_state_hpr; y comes back chunked."""
    import torch
    import mamba_hip
    import oracle
    b, nch, q, h, p, n = 2, 3, 64, 4, 64, 128
    inp = ssd2_inputs(seed=17, b=b, l=nch * q, h=h, p=p, g=1, n=n, h0=True)
    init = (0.1 * np.random.default_rng(18).standard_normal((h, p, n))).astype(np.float32)
    t = _to_dev(inp)
    exp = lambda a: a.repeat_interleave(h, dim=2).reshape(b, nch, q, h, n)  # noqa: E731
    si = mamba_hip.Mamba2SsdInput(
        x_bnlhp=t["x"].reshape(b, nch, q, h, p), dt_bnlh=t["dt"].reshape(b, nch, q, h), a_decay_h=t["A"],
        b_bnlhr=exp(t["B"]), c_bnlhr=exp(t["C"]), d_h=t["D"], initial_state_bhpr=t["h0"],
        init_state_hpr=torch.from_numpy(init).cuda())
    path = mamba_hip.Mamba2SsdPath(mamba_hip.Mamba2SsdPath.SERIAL_RECALCULATED, q)
    y, hT = si.run(path)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (b, nch, q, h, p) and tuple(hT.shape) == (b, h, p, n)
    xr, Br, Cr = bf16_round(inp["x"]), bf16_round(inp["B"]), bf16_round(inp["C"])
    yr, hr = oracle.ssd2(xr, inp["dt"], inp["A"], Br, Cr, inp["D"], inp["h0"], init, chunk=q)
    np.testing.assert_allclose(y.float().cpu().numpy().reshape(b, nch * q, h, p), yr, **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **BF16_TOL)


def test_mamba2_ssd_path_default_chunk():
    """Mamba2SsdPath with no chunk length takes optimal_chunk_len
    (ssd_path.rs:109-114, 139-155): 96 for r=128, p=64 and 64 for r=p=64.  The
    SSD called with chunk_len=None chunks at that length, and the result is
    the oracle's at chunk 96."""
    import torch
    import mamba_hip
    P = mamba_hip.Mamba2SsdPath
    path = P()
    assert path.kind == P.SERIAL_RECALCULATED and path.chunk_len() is None
    assert path.chunk_len_or_optimal(128, 64) == 96 == P.optimal_chunk_len(128, 64)
    assert path.chunk_len_or_optimal(64, 64) == 64
    assert P.optimal_chunk_len(16, 16) == 32 and P.optimal_chunk_len(4096, 4096) == 512
    assert P(P.MINIMAL, 48).chunk_len_or_optimal(128, 64) == 48
    inp = ssd2_inputs(seed=19, b=1, l=300, h=4, p=64, g=1, n=128, h0=True)
    t = _to_dev(inp)
    assert mamba_hip.ssd2_fast_path(t["x"], t["dt"], t["A"], t["B"], t["C"], chunk_len=None)
    y, hT = mamba_hip.ssd2_fwd(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["h0"], chunk_len=None)
    torch.cuda.synchronize()
    yr, hr = _oracle(inp, 96, "bf16")
    np.testing.assert_allclose(y.float().cpu().numpy(), yr, **BF16_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **BF16_TOL)
