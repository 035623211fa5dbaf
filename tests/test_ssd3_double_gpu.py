"""Mamba-3 double-SSD seam: mamba_ssd3_double_fwd (C ABI) vs the CPU oracle
(oracle.ssd3_double, the double serial K1-K5 restatement pinned by the token
recurrence and by the single-SSD oracle at unit coefficients), on the generic
and the MFMA paths; and the double pathway's two seam calls against one
single-SSD call (the single == double identity of the Mamba-3 forward).
f32 at rtol 1e-4, bf16 I/O at rtol 2e-2 / atol 1e-2."""

import numpy as np
import pytest

from inputs import bf16_round, ssd3_inputs

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=2e-5)
BF16_TOL = dict(rtol=2e-2, atol=1e-2)
# bf16 I/O: the state update's operands (decay-weighted v, B) enter the MFMAs
# in bf16 and, with no dt-sized scale column, v keeps its full magnitude, so
# the f32 states carry bf16 operand rounding and are held to the bf16 bar.
BF16_STATE_TOL = BF16_TOL


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


CASES = [
    # (b, l, m, h, p, n, chunk, io)
    (2, 64, 1, 3, 16, 8, 16, "f32"),      # SISO
    (1, 50, 2, 2, 8, 12, 8, "f32"),       # ragged seqlen
    (2, 40, 4, 2, 16, 16, 8, "f32"),      # MIMO 4
    (1, 150, 1, 2, 64, 128, 64, "bf16"),  # MFMA path, SISO, ragged
    (2, 96, 2, 2, 64, 128, 32, "bf16"),   # MFMA path, MIMO 2
    (1, 70, 4, 3, 64, 128, 32, "bf16"),   # MFMA path, MIMO 4, ragged
]


@pytest.mark.parametrize("case", CASES)
def test_ssd3_double_matches_oracle(case):
    import torch
    import mamba_hip
    import oracle
    b, l, m, h, p, n, q, io = case
    d = ssd3_inputs(100 + sum(case[:6]), b, l, m, h, p, n)
    dt = torch.float32 if io == "f32" else torch.bfloat16
    v, B, C = (d[k] if io == "f32" else bf16_round(d[k]) for k in ("v", "B", "C"))
    args = (_t(v, dt), _t(d["da"]), _t(B, dt), _t(C, dt))
    assert mamba_hip.ssd3_double_fast_path(*args, chunk_len=q) == (io == "bf16")
    y, hT = mamba_hip.ssd3_double_fwd(*args, _t(d["h0"]), chunk_len=q)
    torch.cuda.synchronize()
    yr, hr = oracle.ssd3_double(v, d["da"], B, C, d["h0"], chunk=q)
    if io == "f32":
        np.testing.assert_allclose(y.cpu().numpy(), yr, **F32_TOL)
        np.testing.assert_allclose(hT.cpu().numpy(), hr, **F32_TOL)
    else:
        np.testing.assert_allclose(y.float().cpu().numpy(), yr, **BF16_TOL)
        np.testing.assert_allclose(hT.cpu().numpy(), hr, **BF16_STATE_TOL)
        # the generic kernels agree with the fast path on the same bf16 inputs
        yg, hg = mamba_hip.ssd3_double_fwd(*args, _t(d["h0"]), chunk_len=q, generic=True)
        np.testing.assert_allclose(y.float().cpu().numpy(), yg.float().cpu().numpy(), **BF16_TOL)
        np.testing.assert_allclose(hT.cpu().numpy(), hg.cpu().numpy(), **BF16_STATE_TOL)


def test_ssd3_double_groups_null_state_and_input_run():
    """ngroups < nheads, a NULL initial state, and Mamba3DoubleSsdInput.run
    with the learnable init_state_hpr added to the initial state."""
    import torch
    import mamba_hip
    import oracle
    b, l, m, h, p, n = 2, 33, 2, 4, 8, 8
    d = ssd3_inputs(41, b, l, m, h, p, n)
    Bg, Cg = d["B"][:, :, :, :2], d["C"][:, :, :, :2]
    Bh, Ch = np.repeat(Bg, 2, axis=3), np.repeat(Cg, 2, axis=3)
    y, hT = mamba_hip.ssd3_double_fwd(_t(d["v"]), _t(d["da"]), _t(Bg), _t(Cg), None, chunk_len=8)
    torch.cuda.synchronize()
    yr, hr = oracle.ssd3_double(d["v"], d["da"], Bh, Ch, None, chunk=8)
    np.testing.assert_allclose(y.cpu().numpy(), yr, **F32_TOL)
    np.testing.assert_allclose(hT.cpu().numpy(), hr, **F32_TOL)
    init = (0.1 * np.random.default_rng(3).standard_normal((h, p, n))).astype(np.float32)
    inp = mamba_hip.Mamba3DoubleSsdInput(_t(d["v"]), _t(d["da"]), _t(Bg), _t(Cg), _t(d["h0"]), _t(init))
    y2, h2 = inp.run(chunk_len=16)
    torch.cuda.synchronize()
    yr2, hr2 = oracle.ssd3_double(d["v"], d["da"], Bh, Ch, d["h0"] + init[None], chunk=16)
    np.testing.assert_allclose(y2.cpu().numpy(), yr2, **F32_TOL)
    np.testing.assert_allclose(h2.cpu().numpy(), hr2, **F32_TOL)


@pytest.mark.parametrize("io,m", [("f32", 2), ("bf16", 1), ("bf16", 4)])
def test_double_pathway_equals_single(io, m):
    """forward_double_ssd's two seam calls (double_ssd/double_ssd/mod.rs:254-283):
    gamma_t v_t with B_t from the cached state, plus beta_t v_{t-1} with B_{t-1}
    (the cache's v_prev / K_prev at t = 0) from zero, equal one single-SSD
    call with scale_t = gamma_t + (1 - lam_{t+1}) dt_{t+1} from the seeded
    state h0 + (dt_0 - gamma_0) sum_m v_prev[m] (x) K_prev[m]
    (single_ssd/single_ssd/mod.rs:129-225): outputs and final states."""
    import torch
    import mamba_hip
    b, l, h = 2, 77, 2
    p, n, q = (16, 16, 16) if io == "f32" else (64, 128, 32)
    d = ssd3_inputs(60 + m, b, l, m, h, p, n)
    rng = np.random.default_rng(61 + m)
    v_prev = rng.standard_normal((b, m, h, p)).astype(np.float32)
    k_prev = (rng.standard_normal((b, m, h, n)) / np.sqrt(n)).astype(np.float32)
    v, B, C = d["v"], d["B"], d["C"]
    if io == "bf16":
        v, B, C, v_prev, k_prev = map(bf16_round, (v, B, C, v_prev, k_prev))
    gamma = d["gamma"].astype(np.float64)
    beta = d["beta"]
    v_shift = np.concatenate([v_prev[:, None], v[:, :-1]], 1)
    b_shift = np.concatenate([k_prev[:, None], B[:, :-1]], 1)
    v_gamma = (gamma[:, :, None, :, None] * v).astype(np.float32)
    v_beta = (beta[:, :, None, :, None] * v_shift).astype(np.float32)
    dt = torch.float32 if io == "f32" else torch.bfloat16
    yg, hg = mamba_hip.ssd3_double_fwd(_t(v_gamma, dt), _t(d["da"]), _t(B, dt), _t(C, dt), _t(d["h0"]),
                                       chunk_len=q)
    yb, hb = mamba_hip.ssd3_double_fwd(_t(v_beta, dt), _t(d["da"]), _t(b_shift, dt), _t(C, dt),
                                       torch.zeros_like(hg), chunk_len=q)
    seed = (d["dt"][:, 0] - gamma[:, 0])[:, :, None, None] * np.einsum("bmhp,bmhn->bhpn", v_prev, k_prev)
    h0s = (d["h0"] + seed).astype(np.float32)
    ys, hs = mamba_hip.ssd3_fwd(_t(v, dt), _t(d["da"]), _t(B, dt), _t(C, dt), _t(d["gamma"]), _t(d["scale"]),
                                _t(h0s), chunk_len=q)
    torch.cuda.synchronize()
    y_double = yg.float().cpu().numpy() + yb.float().cpu().numpy()
    tol = F32_TOL if io == "f32" else dict(rtol=3e-2, atol=2e-2)  # two bf16-rounded outputs summed
    np.testing.assert_allclose(y_double, ys.float().cpu().numpy(), **tol)
    np.testing.assert_allclose(hg.cpu().numpy() + hb.cpu().numpy(), hs.cpu().numpy(),
                               **(F32_TOL if io == "f32" else BF16_STATE_TOL))
