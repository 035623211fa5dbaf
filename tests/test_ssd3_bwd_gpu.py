"""Mamba-3 SSD backward (mamba_ssd3_bwd, C ABI) against the CPU oracle's
float64 reverse recurrence (oracle.ssd3_bwd, pinned by finite differences in
test_oracle.py): every gradient of the single seam's seven inputs
(src/mamba3/single_ssd/ssd/serial_recalculated/combined_backward.rs:74-536) and
of the double seam's five (unit weights, double_ssd/ssd/serial_recalculated/
combined_backward.rs:98-542), across MIMO ranks, ragged lengths, grouped and
per-head B/C, with the initial state and d(final state) present or absent;
then the autograd node through torch.  f32 gradients within rtol 1e-4 and an
absolute 1e-4 of each gradient's scale."""

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

CASES = [
    # (b, l, m, h, p, g, n, weights, with_h0, with_dfinal)
    (2, 21, 4, 2, 16, 2, 32, True, True, True),     # MIMO 4 (8 steps per chunk), ragged, per-head B / C
    (1, 40, 2, 4, 16, 1, 16, True, False, True),    # MIMO 2, one group
    (2, 13, 1, 3, 8, 3, 32, True, True, False),     # SISO, no d(final state)
    (1, 19, 8, 2, 16, 1, 32, False, True, True),    # MIMO 8, unit weights (the double seam)
    # headdim 64 x dstate 128 with float4-aligned rows: the MFMA kernels
    (1, 70, 4, 2, 64, 2, 128, True, True, True),    # config-4 head shape, per-head B / C
    (2, 37, 2, 4, 64, 1, 128, True, True, True),    # MIMO 2, one group, ragged
    (1, 40, 1, 2, 64, 1, 128, True, False, True),   # SISO (32 steps per chunk)
    (1, 21, 8, 2, 64, 2, 128, False, True, True),   # MIMO 8, unit weights (the double seam)
    (8, 20, 4, 32, 64, 32, 128, True, True, True),  # 512 workgroups: the two-per-CU (128-register) build
]


def _inputs(seed, b, l, m, h, p, g, n, weights, with_h0, with_dfinal):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    d = dict(v=r(b, l, m, h, p), da=(-rng.uniform(0.01, 0.5, (b, l, h))).astype(np.float32),
             B=(r(b, l, m, g, n) / np.sqrt(n)).astype(np.float32), C=(r(b, l, m, g, n) / np.sqrt(n)).astype(np.float32),
             gamma=rng.uniform(0.01, 0.3, (b, l, h)).astype(np.float32) if weights else None,
             scale=rng.uniform(0.02, 0.5, (b, l, h)).astype(np.float32) if weights else None,
             h0=(0.3 * r(b, h, p, n)).astype(np.float32) if with_h0 else None)
    return d, r(b, l, m, h, p), r(b, h, p, n) if with_dfinal else None


def _t(a):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _close(got, want, name):
    scale = float(np.abs(want).max()) or 1.0
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * scale, err_msg=name)


@pytest.mark.parametrize("case", CASES)
def test_ssd3_bwd_matches_oracle(case):
    import torch
    import mamba_hip
    print("ssd3 bwd", case, flush=True)
    d, dy, dF = _inputs(sum(case[:7]), *case)
    out = mamba_hip.ssd3_bwd(_t(dy), _t(d["v"]), _t(d["da"]), _t(d["B"]), _t(d["C"]), _t(d["gamma"]),
                             _t(d["scale"]), _t(d["h0"]), _t(dF))
    torch.cuda.synchronize()
    want = oracle.ssd3_bwd(dy, dF, d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], d["h0"])
    for k, w in (("dv", "dv"), ("dda", "dda"), ("dB", "dB"), ("dC", "dC"), ("d_initial_state", "dh0")):
        _close(out[k].cpu().numpy(), want[w], k)
    if d["gamma"] is not None:
        _close(out["dgamma"].cpu().numpy(), want["dgamma"], "dgamma")
        _close(out["dscale"].cpu().numpy(), want["dscale"], "dscale")
    else:
        assert out["dgamma"] is None and out["dscale"] is None


@pytest.mark.parametrize("p,n", [(16, 32), (64, 128)])
def test_ssd3_bwd_strided_inputs(p, n):
    """The seam's layouts through strides: v and dy as views of a wider row,
    da / gamma / scale as [b, h, l] tensors viewed [b, l, h], B / C as slices
    of one wider row (an odd row length, so at headdim 64 x dstate 128 the
    unaligned rows take the SIMT kernels)."""
    import torch
    import mamba_hip
    b, l, m, h, g = 2, 30, 2, 2, 1
    print("ssd3 bwd strided", p, n, flush=True)
    d, dy, dF = _inputs(7, b, l, m, h, p, g, n, True, True, True)
    wide = torch.zeros((b, l, m, h, p + 4), device="cuda")
    wide[..., :p] = _t(d["v"])
    vv = wide[..., :p]
    bhl = lambda a: _t(np.ascontiguousarray(a.transpose(0, 2, 1))).permute(0, 2, 1)  # noqa: E731
    row = torch.zeros((b, l, m, g, 2 * n + 3), device="cuda")
    row[..., :n] = _t(d["B"])
    row[..., n:2 * n] = _t(d["C"])
    out = mamba_hip.ssd3_bwd(_t(dy), vv, bhl(d["da"]), row[..., :n], row[..., n:2 * n], bhl(d["gamma"]),
                             bhl(d["scale"]), _t(d["h0"]), _t(dF))
    torch.cuda.synchronize()
    want = oracle.ssd3_bwd(dy, dF, d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], d["h0"])
    for k, w in (("dv", "dv"), ("dda", "dda"), ("dB", "dB"), ("dC", "dC"), ("dgamma", "dgamma"),
                 ("dscale", "dscale"), ("d_initial_state", "dh0")):
        _close(out[k].cpu().numpy(), want[w], k)


def test_ssd3_autograd_node():
    """ssd3_autograd: torch's backward through the one-node single SSD (forward
    on the library's forward path) gives the oracle's gradients."""
    import torch
    import mamba_hip
    b, l, m, h, p, g, n = 1, 50, 4, 2, 64, 2, 128
    print("ssd3 autograd", flush=True)
    d, dy, dF = _inputs(9, b, l, m, h, p, g, n, True, True, True)
    ts = {k: _t(v).requires_grad_() for k, v in d.items()}
    y, hT = mamba_hip.ssd3_autograd(ts["v"], ts["da"], ts["B"], ts["C"], ts["gamma"], ts["scale"], ts["h0"],
                                    chunk_len=32)
    loss = (y * _t(dy)).sum() + (hT * _t(dF)).sum()
    loss.backward()
    torch.cuda.synchronize()
    want = oracle.ssd3_bwd(dy, dF, d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], d["h0"])
    for k, w in (("v", "dv"), ("da", "dda"), ("B", "dB"), ("C", "dC"), ("gamma", "dgamma"), ("scale", "dscale"),
                 ("h0", "dh0")):
        _close(ts[k].grad.cpu().numpy(), want[w], k)
