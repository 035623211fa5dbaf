"""Mamba-1 decode step: mamba1_scan_step / mamba_conv1d_step (C ABI) and the
Mamba1 block step against the CPU oracle.  f32: rtol 1e-4 (BASELINE.json
north_star); states compared in every case."""

import numpy as np
import pytest

from inputs import mamba1_inputs

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-4, atol=1e-5)


def _t(a):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n", [16, 32, 64, 5])
def test_scan_step_matches_oracle(n):
    """Several tokens stepped through mamba1_scan_step equal the oracle's step
    (and so the selective scan), with bias + softplus + gate."""
    import torch
    import mamba_hip
    import oracle
    b, d, L = 3, 200, 4  # 200 channels: a ragged last workgroup for every n
    inp = mamba1_inputs(seed=n, b=b, d=d, l=L, n=n, h0=True)
    rng = np.random.default_rng(n)
    bias = (0.3 * rng.standard_normal(d)).astype(np.float32)
    raw = (rng.standard_normal((b, d, L)) - 3).astype(np.float32)
    state = _t(inp["h0"])
    ref_state = inp["h0"]
    A = _t(inp["A"])
    for t in range(L):
        args = [np.ascontiguousarray(inp["u"][:, :, t]), np.ascontiguousarray(raw[:, :, t]),
                np.ascontiguousarray(inp["B"][:, :, t]), np.ascontiguousarray(inp["C"][:, :, t]),
                np.ascontiguousarray(inp["z"][:, :, t])]
        y = mamba_hip.scan_step(_t(args[0]), _t(args[1]), A, _t(args[2]), _t(args[3]), state, D=_t(inp["D"]),
                                z=_t(args[4]), delta_bias=_t(bias), delta_softplus=True)
        torch.cuda.synchronize()
        yr, ref_state = oracle.mamba1_step(args[0], args[1], inp["A"], args[2], args[3], ref_state, inp["D"],
                                           args[4], bias, True)
        print(f"n={n} token {t}", flush=True)
        np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)
        np.testing.assert_allclose(state.cpu().numpy(), ref_state, **TOL)


def test_selective_scan_step_signature_and_strides():
    """Reference signature (no bias/softplus/gate), B/C as strided column views."""
    import torch
    import mamba_hip
    import oracle
    b, d, n = 2, 64, 16
    inp = mamba1_inputs(seed=3, b=b, d=d, l=1, n=n, h0=True)
    u = np.ascontiguousarray(inp["u"][:, :, 0])
    dl = np.ascontiguousarray(inp["delta"][:, :, 0])
    bc = np.concatenate([inp["B"][:, :, 0], inp["C"][:, :, 0]], 1)  # [b, 2n]: B, C as views
    bcd = _t(bc)
    st = _t(inp["h0"])
    y, st2 = mamba_hip.selective_scan_step(_t(dl), _t(inp["A"]), bcd[:, :n], bcd[:, n:], _t(inp["D"]), _t(u), st)
    torch.cuda.synchronize()
    yr, sr = oracle.mamba1_step(u, dl, inp["A"], bc[:, :n], bc[:, n:], inp["h0"], inp["D"])
    assert st2.data_ptr() == st.data_ptr()
    np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)
    np.testing.assert_allclose(st.cpu().numpy(), sr, **TOL)


@pytest.mark.parametrize("k,silu,xdt", [(4, True, "f32"), (3, False, "f32"), (4, True, "bf16"), (1, True, "f32")])
def test_conv1d_step_matches_oracle(k, silu, xdt):
    import torch
    import mamba_hip
    import oracle
    rng = np.random.default_rng(k)
    b, c = 3, 300
    w = rng.standard_normal((c, k)).astype(np.float32)
    bias = rng.standard_normal(c).astype(np.float32)
    st_h = rng.standard_normal((b, c, k)).astype(np.float32)
    st = _t(st_h)
    for t in range(3):
        x = rng.standard_normal((b, c)).astype(np.float32)
        xd = _t(x)
        if xdt == "bf16":
            xd = xd.to(torch.bfloat16)
            x = xd.float().cpu().numpy()
        out = mamba_hip.conv1d_step(xd, st, _t(w), _t(bias), silu=silu)
        torch.cuda.synchronize()
        ref, st_h = oracle.conv1d_step(x, st_h, w, bias, silu)
        np.testing.assert_array_equal(st.cpu().numpy(), st_h)
        np.testing.assert_allclose(out.cpu().numpy(), ref, **TOL)


def _oracle_params(m):
    f = lambda t: None if t is None else t.float().cpu().numpy()  # noqa: E731
    return dict(in_proj_w=f(m.in_proj_w), conv_w=f(m.conv_w), conv_b=f(m.conv_b), x_proj_w=f(m.x_proj_w),
                dt_proj_w=f(m.dt_proj_w), dt_proj_b=f(m.dt_proj_b), A=f(m.A), D=f(m.d), out_proj_w=f(m.out_proj_w))


def test_mamba1_block_step_matches_oracle():
    """Mamba1::step (mamba1.rs:533-612) for three tokens from a zero cache."""
    import torch
    import mamba_hip
    import oracle
    cfg = mamba_hip.Mamba1Config(d_model=64)
    m = cfg.init("cuda", torch.Generator().manual_seed(8))
    p = _oracle_params(m)
    b = 2
    rng = np.random.default_rng(9)
    cache = None
    conv = np.zeros((b, cfg.d_inner, cfg.conv_kernel), np.float32)
    ssm = np.zeros((b, cfg.d_inner, cfg.state_rank), np.float32)
    for t in range(3):
        x = rng.standard_normal((b, 64)).astype(np.float32)
        y, cache = m.step(_t(x), cache)
        torch.cuda.synchronize()
        yr, conv, ssm = oracle.mamba1_block_step(x, p, conv, ssm)
        print(f"token {t}", flush=True)
        np.testing.assert_allclose(cache.conv_bik.cpu().numpy(), conv, **TOL)
        np.testing.assert_allclose(cache.ssm_bir.cpu().numpy(), ssm, **TOL)
        np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)


def test_step_unroll_equals_scan_kernel():
    """Stepping L tokens through mamba1_scan_step reproduces mamba1_scan_fwd's
    outputs and final state (the reference's forward == step unroll)."""
    import torch
    import mamba_hip
    b, d, L, n = 2, 128, 20, 16
    inp = mamba1_inputs(seed=30, b=b, d=d, l=L, n=n, h0=True)
    u, dl, B, C, z = (_t(inp[k]) for k in ("u", "delta", "B", "C", "z"))
    A, D = _t(inp["A"]), _t(inp["D"])
    y_scan, h_scan = mamba_hip.mamba1_scan(u, dl, A, B, C, D, z, initial_state=_t(inp["h0"]))
    st = _t(inp["h0"])
    ys = []
    for t in range(L):
        ys.append(mamba_hip.scan_step(u[:, :, t].contiguous(), dl[:, :, t].contiguous(), A, B[:, :, t],
                                      C[:, :, t], st, D=D, z=z[:, :, t].contiguous()))
    y_step = torch.stack(ys, 2)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y_step.cpu().numpy(), y_scan.cpu().numpy(), **TOL)
    np.testing.assert_allclose(st.cpu().numpy(), h_scan.cpu().numpy(), **TOL)
