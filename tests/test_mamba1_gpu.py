"""Mamba-1 selective scan: libmamba_hip.so (C ABI) vs the f64 CPU oracle.

f32 throughout, so the bar is rtol 1e-4 with a
small atol for outputs near zero; final states are compared in every case."""

import numpy as np
import pytest

from inputs import mamba1_inputs

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-4, atol=2e-5)


def _dev(a):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _oracle(inp, **kw):
    import oracle
    return oracle.mamba1_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                              h0=inp["h0"], **kw)


CASES = [
    # (b, d, l, n)
    (2, 128, 300, 16),    # config-2 shape, reduced; ragged tile
    (1, 96, 64, 16),      # channel count not a multiple of 64
    (2, 64, 33, 32),
    (1, 64, 70, 64),
    (2, 10, 17, 5),       # generic kernel (dstate 5)
    (1, 3, 1, 16),        # single token
]


@pytest.mark.parametrize("case", CASES)
def test_mamba1_scan_matches_oracle(case):
    import torch
    import mamba_hip
    b, d, l, n = case
    inp = mamba1_inputs(seed=sum(case), b=b, d=d, l=l, n=n, h0=True)
    y, hT = mamba_hip.mamba1_scan(_dev(inp["u"]), _dev(inp["delta"]), _dev(inp["A"]), _dev(inp["B"]),
                                  _dev(inp["C"]), _dev(inp["D"]), _dev(inp["z"]),
                                  initial_state=_dev(inp["h0"]))
    torch.cuda.synchronize()
    yr, hr = _oracle(inp)
    np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **TOL)


def test_mamba1_delta_bias_softplus_no_gate():
    """dt_proj bias + softplus (mamba1.rs:391-394), no z gate, no D."""
    import torch
    import mamba_hip
    inp = mamba1_inputs(seed=4, b=2, d=64, l=100, n=16)
    raw = np.random.default_rng(1).standard_normal(inp["u"].shape).astype(np.float32) - 2.0
    bias = np.random.default_rng(2).standard_normal(64).astype(np.float32) * 0.5
    y, hT = mamba_hip.mamba1_scan(_dev(inp["u"]), _dev(raw), _dev(inp["A"]), _dev(inp["B"]), _dev(inp["C"]),
                                  None, None, delta_bias=_dev(bias), delta_softplus=True)
    torch.cuda.synchronize()
    import oracle
    yr, hr = oracle.mamba1_scan(inp["u"], raw, inp["A"], inp["B"], inp["C"], None, None, delta_bias=bias,
                                delta_softplus=True)
    np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **TOL)


@pytest.mark.parametrize("l,pad", [(37, 40), (61, 64), (32, 36)])
def test_mamba1_padded_rows(l, pad):
    """Time-contiguous rows with a padded row stride (16-byte aligned) and a
    sequence that ends inside a 16-byte piece: the tiled path's last-tile
    masking.  Bias + softplus + gate + D; y's padding must stay untouched."""
    import torch
    import mamba_hip
    import oracle
    b, d, n = 2, 130, 16
    inp = mamba1_inputs(seed=l, b=b, d=d, l=l, n=n, h0=True)
    raw = (np.random.default_rng(l).standard_normal((b, d, l)) - 2.0).astype(np.float32)
    bias = (0.5 * np.random.default_rng(l + 1).standard_normal(d)).astype(np.float32)

    def padded(a, fill=0.0):
        t = torch.full((b, d, pad), fill, device="cuda")
        t[:, :, :l] = _dev(a)
        return t[:, :, :l]

    y = padded(np.zeros((b, d, l), np.float32), fill=7.0)
    _, hT = mamba_hip.mamba1_scan(padded(inp["u"]), padded(raw), _dev(inp["A"]), _dev(inp["B"]), _dev(inp["C"]),
                                  _dev(inp["D"]), padded(inp["z"]), delta_bias=_dev(bias), delta_softplus=True,
                                  initial_state=_dev(inp["h0"]), y=y)
    torch.cuda.synchronize()
    yr, hr = oracle.mamba1_scan(inp["u"], raw, inp["A"], inp["B"], inp["C"], inp["D"], inp["z"], delta_bias=bias,
                                delta_softplus=True, h0=inp["h0"])
    np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **TOL)
    full = y.as_strided((b, d, pad), y.stride()).cpu().numpy()
    assert (full[:, :, l:] == 7.0).all()


def test_mamba1_reference_signature_and_layouts():
    """Mamba1::selective_scan(delta [s,b,d], a, b [b,s,r], c [s,b,r], d, u [b,s,d], init)
    (mamba1.rs:422-430) gives the channel-major result transposed."""
    import torch
    import mamba_hip
    inp = mamba1_inputs(seed=6, b=2, d=64, l=80, n=16, h0=True)
    u_bsd = _dev(inp["u"].transpose(0, 2, 1))
    delta_sbd = _dev(inp["delta"].transpose(2, 0, 1))
    b_bsr = _dev(inp["B"].transpose(0, 2, 1))
    c_sbr = _dev(inp["C"].transpose(2, 0, 1))
    y, hT = mamba_hip.selective_scan(delta_sbd, _dev(inp["A"]), b_bsr, c_sbr, _dev(inp["D"]), u_bsd,
                                     _dev(inp["h0"]))
    torch.cuda.synchronize()
    yr, hr = _oracle(dict(inp, z=None))
    np.testing.assert_allclose(y.cpu().numpy().transpose(0, 2, 1), yr, **TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **TOL)


def test_mamba1_golden_fixture():
    import os
    import torch
    import mamba_hip
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "mamba1_cfg2_small.npz"))
    y, hT = mamba_hip.mamba1_scan(_dev(f["u"]), _dev(f["delta"]), _dev(f["A"]), _dev(f["B"]), _dev(f["C"]),
                                  _dev(f["D"]), _dev(f["z"]), initial_state=_dev(f["h0"]))
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), f["y"], **TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), f["final_state"], **TOL)


def test_mamba1_split_equals_full():
    """Cache continuity (src/mamba1/mamba1/tests.rs:384-429): two calls threading
    the final state reproduce one call over the whole sequence."""
    import torch
    import mamba_hip
    inp = mamba1_inputs(seed=8, b=1, d=64, l=96, n=16, h0=True)
    t = {k: _dev(v) for k, v in inp.items()}
    y, hT = mamba_hip.mamba1_scan(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["z"],
                                  initial_state=t["h0"])
    s = 41
    ya, ha = mamba_hip.mamba1_scan(t["u"][..., :s], t["delta"][..., :s], t["A"], t["B"][..., :s],
                                   t["C"][..., :s], t["D"], t["z"][..., :s], initial_state=t["h0"])
    yb, hb = mamba_hip.mamba1_scan(t["u"][..., s:], t["delta"][..., s:], t["A"], t["B"][..., s:],
                                   t["C"][..., s:], t["D"], t["z"][..., s:], initial_state=ha)
    torch.cuda.synchronize()
    np.testing.assert_allclose(torch.cat([ya, yb], -1).cpu().numpy(), y.cpu().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(hb.cpu().numpy(), hT.cpu().numpy(), rtol=1e-5, atol=1e-6)


def test_mamba1_config2_full_size():
    """BASELINE.json configs[2] at its full size (8 x 5120 channels x 2048
    tokens, dstate 16, f32, z gate, D = 1): the benched kernel against the f64
    oracle at north_star's f32 bar, outputs and final states."""
    import torch
    import mamba_hip
    b, d, l, n = 8, 5120, 2048, 16
    print(f"mamba1 config 2 full size {b}x{d}x{l}", flush=True)
    inp = mamba1_inputs(seed=2048, b=b, d=d, l=l, n=n)
    y, hT = mamba_hip.mamba1_scan(_dev(inp["u"]), _dev(inp["delta"]), _dev(inp["A"]), _dev(inp["B"]),
                                  _dev(inp["C"]), _dev(inp["D"]), _dev(inp["z"]))
    torch.cuda.synchronize()
    y, hT = y.cpu().numpy(), hT.cpu().numpy()
    yr, hr = _oracle(inp)
    for i in range(b):
        np.testing.assert_allclose(y[i], yr[i], err_msg=f"y[{i}]", **TOL)
    np.testing.assert_allclose(hT, hr, **TOL)
