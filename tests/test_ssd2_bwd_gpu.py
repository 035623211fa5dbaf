"""Mamba-2 SSD backward (mamba_ssd2_bwd, C ABI) against the CPU oracle's
float64 reverse recurrence (oracle.ssd2_bwd, pinned by finite differences in
test_oracle.py): every gradient of the seam's seven inputs
(src/mamba2/ssd/serial_recalculated/combined_backward.rs:126-593), across
ragged lengths, grouped and per-head B/C, the config-1 head shape, and with D,
the initial state and d(final state) present or absent; then the autograd
node (the reference's Autodiff arm, backward.rs:29-321) through torch.
f32 gradients within rtol 1e-4 and an absolute 1e-4 of each gradient's scale."""

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

CASES = [
    # (b, l, h, p, g, n, with_D, with_h0, with_dfinal)
    (2, 37, 4, 16, 2, 16, True, True, True),     # ragged last chunk, two groups
    (1, 100, 2, 64, 1, 128, True, True, True),   # config-1 head shape (P 64, N 128)
    (2, 64, 4, 32, 4, 64, False, False, True),   # per-head B / C (ngroups = nheads), no D / h0
    (1, 45, 3, 8, 1, 32, True, False, False),    # no d(final state)
    # headdim 64 x dstate 128 with float4-aligned rows: the MFMA kernels
    (2, 200, 4, 64, 2, 128, True, True, True),   # seven chunks, ragged tail, two groups
    (1, 64, 2, 64, 2, 128, False, False, False), # per-head B / C, nothing optional
]


def _inputs(seed, b, l, h, p, g, n, with_D, with_h0, with_dfinal):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    d = dict(x=r(b, l, h, p), dt=rng.uniform(0.01, 0.3, (b, l, h)).astype(np.float32),
             A=(-np.exp(rng.uniform(0.0, np.log(8.0), h))).astype(np.float32),
             B=(r(b, l, g, n) / np.sqrt(n)).astype(np.float32), C=(r(b, l, g, n) / np.sqrt(n)).astype(np.float32),
             D=r(h) if with_D else None, h0=(0.3 * r(b, h, p, n)).astype(np.float32) if with_h0 else None)
    return d, r(b, l, h, p), r(b, h, p, n) if with_dfinal else None


def _t(a):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _close(got, want, name):
    scale = float(np.abs(want).max()) or 1.0
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * scale, err_msg=name)


@pytest.mark.parametrize("case", CASES)
def test_ssd2_bwd_matches_oracle(case):
    import torch
    import mamba_hip
    print("ssd2 bwd", case, flush=True)
    d, dy, dF = _inputs(sum(case[:6]), *case)
    out = mamba_hip.ssd2_bwd(_t(dy), _t(d["x"]), _t(d["dt"]), _t(d["A"]), _t(d["B"]), _t(d["C"]), _t(d["D"]),
                             _t(d["h0"]), _t(dF))
    torch.cuda.synchronize()
    want = oracle.ssd2_bwd(dy, dF, d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["h0"])
    for k, w in (("dx", "dx"), ("ddt", "ddt"), ("dA", "dA"), ("dB", "dB"), ("dC", "dC"),
                 ("d_initial_state", "dh0")):
        _close(out[k].cpu().numpy(), want[w], k)
    if d["D"] is not None:
        _close(out["dD"].cpu().numpy(), want["dD"], "dD")
    else:
        assert out["dD"] is None


@pytest.mark.parametrize("p,n", [(16, 32), (64, 128)])
def test_ssd2_bwd_strided_inputs(p, n):
    """The seam's layouts through strides: x and dy as [b, l, h, p] views of a
    wider row, dt as a [b, h, l] tensor viewed [b, l, h] (the reference's
    dt_bhnl), B / C as slices of one xBC row (an odd row length, so at
    headdim 64 x dstate 128 the unaligned rows take the SIMT kernels)."""
    import torch
    import mamba_hip
    print("ssd2 bwd strided", p, n, flush=True)
    b, l, h, g = 2, 50, 4, 2
    d, dy, dF = _inputs(5, b, l, h, p, g, n, True, True, True)
    wide = torch.zeros((b, l, h, p + 8), device="cuda")
    wide[..., :p] = _t(d["x"])
    xv = wide[..., :p]
    dt_bhl = _t(np.ascontiguousarray(d["dt"].transpose(0, 2, 1)))
    dtv = dt_bhl.permute(0, 2, 1)
    xbc = torch.zeros((b, l, 2 * g * n + 3), device="cuda")
    xbc[..., :g * n] = _t(d["B"]).reshape(b, l, g * n)
    xbc[..., g * n:2 * g * n] = _t(d["C"]).reshape(b, l, g * n)
    Bv = xbc[..., :g * n].unflatten(2, (g, n))
    Cv = xbc[..., g * n:2 * g * n].unflatten(2, (g, n))
    out = mamba_hip.ssd2_bwd(_t(dy), xv, dtv, _t(d["A"]), Bv, Cv, _t(d["D"]), _t(d["h0"]), _t(dF))
    torch.cuda.synchronize()
    want = oracle.ssd2_bwd(dy, dF, d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["h0"])
    for k, w in (("dx", "dx"), ("ddt", "ddt"), ("dB", "dB"), ("dC", "dC"), ("dD", "dD")):
        _close(out[k].cpu().numpy(), want[w], k)


@pytest.mark.parametrize("io", ["f32", "bf16"])
def test_ssd2_autograd_node(io):
    """ssd2_autograd: torch's backward through the one-node SSD (forward on the
    library's forward path, bf16 on its MFMA path) gives the oracle's
    gradients of the same inputs (bf16 ones as the values the kernels read)."""
    import torch
    import mamba_hip
    b, l, h, p, g, n = 2, 70, 4, 64, 1, 128
    d, dy, dF = _inputs(9, b, l, h, p, g, n, True, True, True)
    tdt = torch.bfloat16 if io == "bf16" else torch.float32
    x = _t(d["x"]).to(tdt).requires_grad_()
    B = _t(d["B"]).to(tdt).requires_grad_()
    C = _t(d["C"]).to(tdt).requires_grad_()
    dt, A, D, h0 = (_t(d[k]).requires_grad_() for k in ("dt", "A", "D", "h0"))
    y, hT = mamba_hip.ssd2_autograd(x, dt, A, B, C, D, h0, chunk_len=64)
    loss = (y.float() * _t(dy)).sum() + (hT * _t(dF)).sum()
    loss.backward()
    torch.cuda.synchronize()
    xs, Bs, Cs = (t.detach().float().cpu().numpy() for t in (x, B, C))
    # a bf16 y receives its gradient in bf16: the node's dy is dy rounded to bf16
    dyv = _t(dy).to(tdt).float().cpu().numpy()
    want = oracle.ssd2_bwd(dyv, dF, xs, d["dt"], d["A"], Bs, Cs, d["D"], d["h0"])
    # gradients are f32 from the kernels; bf16 parameters receive them rounded to bf16
    tol = (lambda a, w, nm: _close(a, w, nm)) if io == "f32" else \
        (lambda a, w, nm: np.testing.assert_allclose(a, w, rtol=1e-2, atol=1e-2 * float(np.abs(w).max()), err_msg=nm))
    tol(x.grad.float().cpu().numpy(), want["dx"], "dx")
    tol(B.grad.float().cpu().numpy(), want["dB"], "dB")
    tol(C.grad.float().cpu().numpy(), want["dC"], "dC")
    _close(dt.grad.cpu().numpy(), want["ddt"], "ddt")
    _close(A.grad.cpu().numpy(), want["dA"], "dA")
    _close(D.grad.cpu().numpy(), want["dD"], "dD")
    _close(h0.grad.cpu().numpy(), want["dh0"], "dh0")
