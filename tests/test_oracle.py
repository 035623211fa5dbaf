"""Pins the CPU oracle (oracle/) without running the reference.

The reference is Rust over Burn; neither a Rust toolchain nor Burn's sources
exist here and it ships no golden vectors, so each oracle function is checked
against an independent formulation that a plausible slip (dropped term, wrong
sign, off-by-one in the causal mask, transposed operand) would break:
  * three algebraically distinct SSD forms (serial K1-K5, minimal/segsum,
    token recurrence) must agree (the reference's own paths_agree tests,
    src/mamba2/ssd/ssd_path/tests.rs:184-336);
  * closed forms: A = 0, dt = 1 reduces the SSD to causal linear attention
    y = tril(C B^T) X + D X (numpy matmuls); delta = 0 makes the Mamba-1 scan
    y = D u; N = 1 with constant delta is a first-order IIR filter
    (scipy.signal.lfilter);
  * invariants: chunk-length independence; zero-dt padding is an identity
    (src/mamba2/mamba2.rs:703-706); split == full (cache continuity); the
    Mamba-1 block forward equals its step unrolled token by token, from zero
    and from random caches (src/mamba1/mamba1/tests.rs:216-372);
  * Mamba-3: the merged single-SSD equals the explicit two-term trapezoid
    recurrence (src/mamba3/mamba3.rs:14-26), and lambda = 1 collapses it to
    Mamba-2.
"""

import numpy as np
import pytest

import oracle
from inputs import mamba1_inputs, softplus, ssd2_inputs, ssd2_test_inputs, ssd3_inputs

SHAPES = [(2, 12, 2, 8, 2, 8, 4), (2, 12, 4, 8, 4, 8, 4), (2, 4, 2, 8, 1, 8, 4), (1, 37, 4, 8, 2, 8, 8)]


@pytest.mark.parametrize("shape", SHAPES)
def test_ssd2_three_forms_agree(shape):
    b, l, h, p, g, n, q = shape
    inp = ssd2_test_inputs(1, b, l, h, p, g, n)
    args = (inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"])
    ys, hs = oracle.ssd2(*args, chunk=q, form="serial")
    ym, hm = oracle.ssd2(*args, chunk=q, form="minimal")
    yr, hr = oracle.ssd2(*args, form="recurrent")
    for a, r in ((ys, yr), (ym, yr), (hs, hr), (hm, hr)):
        np.testing.assert_allclose(a, r, rtol=1e-6, atol=1e-6)
    # the f32 restatement (the reference's own arithmetic width) stays within 1e-4
    y32, h32 = oracle.ssd2(*args, chunk=q, form="serial", prec=32)
    np.testing.assert_allclose(y32, yr, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(h32, hr, rtol=1e-4, atol=1e-4)


def test_ssd2_linear_attention_closed_form():
    b, l, h, p, g, n = 2, 40, 3, 5, 1, 6
    rng = np.random.default_rng(5)
    x = rng.standard_normal((b, l, h, p)).astype(np.float32)
    B = rng.standard_normal((b, l, g, n)).astype(np.float32)
    C = rng.standard_normal((b, l, g, n)).astype(np.float32)
    D = rng.standard_normal(h).astype(np.float32)
    dt = np.ones((b, l, h), np.float32)
    A = np.zeros(h, np.float32)
    for form in ("serial", "minimal", "recurrent"):
        y, hT = oracle.ssd2(x, dt, A, B, C, D, chunk=8, form=form)
        for bi in range(b):
            M = np.tril(C[bi, :, 0].astype(np.float64) @ B[bi, :, 0].astype(np.float64).T)
            for hi in range(h):
                ref = M @ x[bi, :, hi].astype(np.float64) + D[hi] * x[bi, :, hi]
                np.testing.assert_allclose(y[bi, :, hi], ref, rtol=1e-5, atol=1e-5)
                sref = x[bi, :, hi].astype(np.float64).T @ B[bi, :, 0].astype(np.float64)
                np.testing.assert_allclose(hT[bi, hi], sref, rtol=1e-5, atol=1e-5)


def test_ssd2_chunk_independence_and_padding():
    inp = ssd2_inputs(2, b=2, l=70, h=3, p=8, g=1, n=8, h0=True)
    args = (inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"])
    y0, h0 = oracle.ssd2(*args, chunk=70, form="serial")
    for q in (1, 7, 16, 64, 128):
        y, hT = oracle.ssd2(*args, chunk=q, form="serial")
        np.testing.assert_allclose(y, y0, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(hT, h0, rtol=1e-6, atol=1e-6)
    # zero-dt tokens appended: identity on the state, y there is D*x
    pad = {k: (np.concatenate([v, np.zeros_like(v[:, :5])], 1) if k in ("x", "dt", "B", "C") else v)
           for k, v in inp.items()}
    y2, h2 = oracle.ssd2(pad["x"], pad["dt"], pad["A"], pad["B"], pad["C"], pad["D"], pad["h0"], chunk=16)
    np.testing.assert_allclose(h2, h0, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(y2[:, :70], y0, rtol=1e-6, atol=1e-6)


def test_ssd2_split_equals_full_and_init_hpr():
    inp = ssd2_inputs(3, b=1, l=50, h=2, p=4, g=1, n=4, h0=True)
    full = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"], chunk=8)
    s = 21
    ya, ha = oracle.ssd2(*(inp[k][:, :s] for k in ("x", "dt")), inp["A"], inp["B"][:, :s], inp["C"][:, :s],
                         inp["D"], inp["h0"], chunk=8)
    yb, hb = oracle.ssd2(*(inp[k][:, s:] for k in ("x", "dt")), inp["A"], inp["B"][:, s:], inp["C"][:, s:],
                         inp["D"], ha, chunk=8)
    np.testing.assert_allclose(np.concatenate([ya, yb], 1), full[0], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(hb, full[1], rtol=1e-6, atol=1e-6)
    # learnable init state adds to h0 (minimal.rs:316-328)
    init = np.random.default_rng(4).standard_normal((2, 4, 4)).astype(np.float32)
    y1, h1 = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"], init, chunk=8)
    y2, h2 = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"] + init[None], chunk=8)
    np.testing.assert_allclose(y1, y2, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(h1, h2, rtol=1e-6, atol=1e-6)


def test_ssd2_golden_fixture_regression():
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "ssd2_cfg0_small.npz"))
    y, hT = oracle.ssd2(f["x"], f["dt"], f["A"], f["B"], f["C"], f["D"], f["h0"], chunk=int(f["chunk"]))
    np.testing.assert_allclose(y, f["y"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(hT, f["final_state"], rtol=1e-6, atol=1e-6)
    yr, hr = oracle.ssd2(f["x"], f["dt"], f["A"], f["B"], f["C"], f["D"], f["h0"], form="recurrent")
    np.testing.assert_allclose(yr, f["y"], rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------- Mamba-1 --

def _scan_loop(u, delta, A, B, C, D, z, h0):
    b, d, l = u.shape
    n = A.shape[1]
    y = np.zeros((b, d, l))
    h = np.zeros((b, d, n)) if h0 is None else h0.astype(np.float64).copy()
    for t in range(l):
        dl = delta[:, :, t].astype(np.float64)
        a = np.exp(dl[:, :, None] * A[None].astype(np.float64))
        h = h * a + (dl[:, :, None] * B[:, None, :, t]) * u[:, :, t, None]
        y[:, :, t] = (h * C[:, None, :, t]).sum(-1) + D[None] * u[:, :, t]
    if z is not None:
        y = y * (z / (1 + np.exp(-z.astype(np.float64))))
    return y, h


def test_mamba1_matches_vectorised_loop():
    inp = mamba1_inputs(1, b=2, d=5, l=33, n=4, h0=True)
    y, hT = oracle.mamba1_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                               h0=inp["h0"])
    yr, hr = _scan_loop(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"], inp["h0"])
    np.testing.assert_allclose(y, yr, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(hT, hr, rtol=1e-5, atol=1e-6)


def test_mamba1_closed_forms():
    from scipy.signal import lfilter
    inp = mamba1_inputs(2, b=1, d=3, l=64, n=1)
    # delta = 0: the state stays at h0 and y = C_t . h0 + D*u
    h0 = np.full((1, 3, 1), 0.5, np.float32)
    y, hT = oracle.mamba1_scan(inp["u"], np.zeros_like(inp["delta"]), inp["A"], inp["B"], inp["C"],
                               inp["D"], h0=h0)
    ref = 0.5 * inp["C"][:, 0][:, None, :] + inp["D"][None, :, None] * inp["u"]
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(hT, h0, rtol=0, atol=0)
    # N = 1, constant delta: h_t = a h_{t-1} + delta B_t u_t is an IIR filter
    dl = np.full_like(inp["delta"], 0.07)
    y, hT = oracle.mamba1_scan(inp["u"], dl, inp["A"], inp["B"], inp["C"], None)
    for d in range(3):
        a = np.exp(0.07 * inp["A"][d, 0])
        hseq = lfilter([1.0], [1.0, -a], 0.07 * inp["B"][0, 0] * inp["u"][0, d])
        np.testing.assert_allclose(y[0, d], hseq * inp["C"][0, 0], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(hT[0, d, 0], hseq[-1], rtol=1e-5)


def test_mamba1_step_unroll_equals_scan():
    inp = mamba1_inputs(3, b=2, d=4, l=9, n=3, h0=True)
    y, hT = oracle.mamba1_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                               h0=inp["h0"])
    st = inp["h0"]
    for t in range(9):
        ys, st = oracle.mamba1_step(inp["u"][:, :, t], inp["delta"][:, :, t], inp["A"], inp["B"][:, :, t],
                                    inp["C"][:, :, t], st, inp["D"], inp["z"][:, :, t])
        np.testing.assert_allclose(ys, y[:, :, t], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(st, hT, rtol=1e-5, atol=1e-6)


def test_mamba1_delta_bias_softplus():
    inp = mamba1_inputs(4, b=1, d=3, l=8, n=2)
    bias = np.array([0.1, -0.2, 0.3], np.float32)
    raw = np.random.default_rng(0).standard_normal(inp["u"].shape).astype(np.float32)
    y1, h1 = oracle.mamba1_scan(inp["u"], raw, inp["A"], inp["B"], inp["C"], inp["D"], delta_bias=bias,
                                delta_softplus=True)
    dl = np.log1p(np.exp(raw.astype(np.float64) + bias[None, :, None])).astype(np.float32)
    y2, h2 = oracle.mamba1_scan(inp["u"], dl, inp["A"], inp["B"], inp["C"], inp["D"])
    np.testing.assert_allclose(y1, y2, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------- Mamba-2 step() ----

def _silu(v):
    return v / (1 + np.exp(-v))


def test_mamba2_step_ssm_closed_form():
    """conv + SiLU + softplus + state update + readout + gated RMSNorm, from
    the formulas of mamba2.rs:865-995 written independently in numpy."""
    rng = np.random.default_rng(9)
    b, H, P, G, N, K = 2, 4, 8, 2, 6, 4
    d_inner, conv_dim = H * P, H * P + 2 * G * N
    zx = rng.standard_normal((b, d_inner + conv_dim + H)).astype(np.float32)
    conv_state = rng.standard_normal((b, conv_dim, K)).astype(np.float32)
    conv_w = rng.standard_normal((conv_dim, K)).astype(np.float32) * 0.5
    conv_b = rng.standard_normal(conv_dim).astype(np.float32) * 0.1
    dt_bias = rng.standard_normal(H).astype(np.float32)
    A = -np.exp(rng.uniform(0, 2, H)).astype(np.float32)
    D = rng.standard_normal(H).astype(np.float32)
    nw = rng.standard_normal(d_inner).astype(np.float32)
    ss = rng.standard_normal((b, H, P, N)).astype(np.float32)
    out, cs2, ss2 = oracle.mamba2_step_ssm(zx, conv_state, conv_w, conv_b, dt_bias, A, D, nw, ss, H, P, G, N)
    z, xbc, dtr = zx[:, :d_inner], zx[:, d_inner:d_inner + conv_dim], zx[:, d_inner + conv_dim:]
    win = np.concatenate([conv_state[:, :, 1:], xbc[:, :, None]], 2)
    np.testing.assert_array_equal(cs2, win)
    act = _silu((win.astype(np.float64) * conv_w[None]).sum(-1) + conv_b)
    xs = act[:, :d_inner].reshape(b, H, P)
    Bg = act[:, d_inner:d_inner + G * N].reshape(b, G, N)
    Cg = act[:, d_inner + G * N:].reshape(b, G, N)
    dt = softplus(dtr.astype(np.float64) + dt_bias)
    hpg = H // G
    Bh, Ch = np.repeat(Bg, hpg, 1), np.repeat(Cg, hpg, 1)
    hn = ss * np.exp(dt * A)[:, :, None, None] + dt[:, :, None, None] * Bh[:, :, None, :] * xs[:, :, :, None]
    np.testing.assert_allclose(ss2, hn, rtol=1e-5, atol=1e-6)
    y = (hn * Ch[:, :, None, :]).sum(-1) + D[None, :, None] * xs
    gv = y.reshape(b, d_inner) * _silu(z.astype(np.float64))
    ref = gv / np.sqrt((gv ** 2).mean(-1, keepdims=True) + 8.1584695e-8) * nw
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    # norm_before_gate = true: normalise y first, gate afterwards
    out_nb, _, _ = oracle.mamba2_step_ssm(zx, conv_state, conv_w, conv_b, dt_bias, A, D, nw, ss, H, P, G, N,
                                          norm_before_gate=True)
    yb = y.reshape(b, d_inner)
    ref_nb = yb / np.sqrt((yb ** 2).mean(-1, keepdims=True) + 8.1584695e-8) * nw * _silu(z.astype(np.float64))
    np.testing.assert_allclose(out_nb, ref_nb, rtol=1e-5, atol=1e-6)


def test_mamba2_step_unroll_equals_ssd():
    """forward == step unroll (the reference's src/mamba2/mamba2/tests.rs:202-328)
    at the SSM level: stepping the state update token by token reproduces the
    chunked SSD's final state and outputs."""
    inp = ssd2_inputs(6, b=2, l=11, h=4, p=8, g=2, n=6, h0=True)
    y, hT = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"], chunk=4)
    st = inp["h0"].astype(np.float64)
    hpg = 2
    for t in range(11):
        dt = inp["dt"][:, t].astype(np.float64)
        Bh = np.repeat(inp["B"][:, t], hpg, 1)
        Ch = np.repeat(inp["C"][:, t], hpg, 1)
        st = st * np.exp(dt * inp["A"])[:, :, None, None] + dt[:, :, None, None] * Bh[:, :, None, :] * inp["x"][:, t, :, :, None]
        yt = (st * Ch[:, :, None, :]).sum(-1) + inp["D"][None, :, None] * inp["x"][:, t]
        np.testing.assert_allclose(y[:, t], yt, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(hT, st, rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------- Mamba-3 --

_m3_inputs = ssd3_inputs


def _trapezoid_loop(d, h0_boundary):
    """Explicit trapezoid recurrence (src/mamba3/mamba3.rs:14-26; step form
    double_ssd/double_ssd/mod.rs:713-748): h_t = a_t h_{t-1} + beta_t sum_m
    B_{t-1,m} v_{t-1,m} + gamma_t sum_m B_t,m v_t,m ; y_t,m = C_t,m . h_t."""
    v, B, C = (d[k].astype(np.float64) for k in ("v", "B", "C"))
    b, l, m, h, p = v.shape
    hs = h0_boundary.astype(np.float64).copy()
    y = np.zeros_like(v)
    prev = np.zeros((b, h, p, B.shape[-1]))
    for t in range(l):
        cur = np.einsum("bmhp,bmhn->bhpn", v[:, t], B[:, t])
        hs = np.exp(d["da"][:, t].astype(np.float64))[:, :, None, None] * hs \
            + d["beta"][:, t][:, :, None, None] * prev + d["gamma"][:, t].astype(np.float64)[:, :, None, None] * cur
        y[:, t] = np.einsum("bmhn,bhpn->bmhp", C[:, t], hs)
        prev = cur
    return y, hs


@pytest.mark.parametrize("m", [1, 2, 4])
def test_ssd3_serial_equals_recurrent_and_trapezoid(m):
    d = _m3_inputs(7, b=2, l=19, m=m, h=3, p=4, n=6)
    args = (d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], d["h0"])
    ys, hs = oracle.ssd3(*args, chunk=4)
    yr, hr = oracle.ssd3(*args, form="recurrent")
    np.testing.assert_allclose(ys, yr, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(hs, hr, rtol=1e-6, atol=1e-6)
    # the merged (single-SSD) accumulator h'_t = h_t + (1-lam_{t+1}) dt_{t+1} sum B_t v_t
    # so with zero initial state it must reproduce the explicit trapezoid outputs
    d0 = dict(d, h0=np.zeros_like(d["h0"]))
    y0, _ = oracle.ssd3(d0["v"], d0["da"], d0["B"], d0["C"], d0["gamma"], d0["scale"], d0["h0"], chunk=5)
    yt, _ = _trapezoid_loop(d0, d0["h0"])
    np.testing.assert_allclose(y0, yt, rtol=1e-5, atol=1e-6)


def _double_recurrence(v, da, B, C, h0):
    """The double-SSD seam as a token loop (the textbook SSM recurrence the
    chunked K1-K5 factor): h_t = exp(da_t) h_{t-1} + sum_m v[t, m] (x) B[t, m],
    y[t, m] = C[t, m] . h_t."""
    b, l, m, h, p = v.shape
    hs = np.asarray(h0, np.float64).copy()
    y = np.zeros((b, l, m, h, p))
    for t in range(l):
        hs = np.exp(da[:, t].astype(np.float64))[:, :, None, None] * hs + np.einsum(
            "bmhp,bmhn->bhpn", v[:, t].astype(np.float64), B[:, t].astype(np.float64))
        y[:, t] = np.einsum("bmhn,bhpn->bmhp", C[:, t].astype(np.float64), hs)
    return y, hs


@pytest.mark.parametrize("m,chunk", [(1, 4), (2, 5), (4, 8)])
def test_ssd3_double_equals_recurrence(m, chunk):
    """K1-K5 of the double seam (ragged last chunk included) equal the token
    recurrence, from a non-zero initial state."""
    d = _m3_inputs(17 + m, b=2, l=19, m=m, h=3, p=4, n=6)
    yd, hd = oracle.ssd3_double(d["v"], d["da"], d["B"], d["C"], d["h0"], chunk=chunk)
    yr, hr = _double_recurrence(d["v"], d["da"], d["B"], d["C"], d["h0"])
    np.testing.assert_allclose(yd, yr, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(hd, hr, rtol=1e-10, atol=1e-12)


def test_ssd3_double_is_single_with_unit_coefficients():
    """The double seam is the (pinned) single-SSD seam with scale = gamma = 1:
    weight 1 on every earlier step and on the same step's rank pairs."""
    d = _m3_inputs(23, b=1, l=21, m=2, h=2, p=4, n=5)
    one = np.ones_like(d["gamma"])
    ys, hs = oracle.ssd3(d["v"], d["da"], d["B"], d["C"], one, one, d["h0"], chunk=8)
    yd, hd = oracle.ssd3_double(d["v"], d["da"], d["B"], d["C"], d["h0"], chunk=6)
    np.testing.assert_allclose(yd, ys, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(hd, hs, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("m", [1, 2, 4])
def test_single_ssd_equals_double_ssd_pathway(m):
    """The reference's single == double relation (Mamba-3 forward, single_ssd
    vs double_ssd pathways): the gamma call (gamma_t v_t, B_t, cached state)
    plus the beta call (beta_t v_{t-1}, B_{t-1}, cache's v_prev / K_prev at
    t = 0, zero state) of the double seam equal one single-SSD call from the
    seeded state h0 + (dt_0 - gamma_0) sum_m v_prev (x) K_prev."""
    b, l, h, p, n = 2, 23, 2, 4, 6
    d = _m3_inputs(60 + m, b=b, l=l, m=m, h=h, p=p, n=n)
    rng = np.random.default_rng(61 + m)
    v_prev = rng.standard_normal((b, m, h, p))
    k_prev = rng.standard_normal((b, m, h, n)) / np.sqrt(n)
    v, B, C = d["v"], d["B"], d["C"]
    gamma = d["gamma"].astype(np.float64)
    vs = np.concatenate([v_prev[:, None], v[:, :-1]], 1)
    bs = np.concatenate([k_prev[:, None], B[:, :-1]], 1)
    yg, hg = oracle.ssd3_double(gamma[:, :, None, :, None] * v, d["da"], B, C, d["h0"], chunk=8)
    yb, hb = oracle.ssd3_double(d["beta"][:, :, None, :, None] * vs, d["da"], bs, C, None, chunk=8)
    seed = (d["dt"][:, 0] - gamma[:, 0])[:, :, None, None] * np.einsum("bmhp,bmhn->bhpn", v_prev, k_prev)
    ys, hs = oracle.ssd3(v, d["da"], B, C, d["gamma"], d["scale"], (d["h0"] + seed).astype(np.float32), chunk=8)
    np.testing.assert_allclose(yg + yb, ys, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(hg + hb, hs, rtol=1e-5, atol=1e-6)


def test_ssd3_lambda_one_is_mamba2():
    """lam = 1 removes the beta term: gamma = scale = dt and the single-SSD is
    the Mamba-2 SSD without D (src/mamba3/mamba3.rs:28)."""
    d = _m3_inputs(8, b=1, l=21, m=1, h=2, p=4, n=5, lam=1.0)
    y3, h3 = oracle.ssd3(d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], d["h0"], chunk=8)
    x = d["v"][:, :, 0]
    Bm = d["B"][:, :, 0]
    Cm = d["C"][:, :, 0]
    y2, h2 = oracle.ssd2(x, d["dt"].astype(np.float32), d["A"].astype(np.float32), Bm, Cm, None, d["h0"], chunk=8)
    np.testing.assert_allclose(y3[:, :, 0], y2, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(h3, h2, rtol=1e-5, atol=1e-6)


def test_rmsnorm_and_linear_known_answers():
    """RmsNorm of a constant row c is c / sqrt(c^2 + eps) * w (so +-w for
    |c| >> sqrt(eps)); a row and its negation normalise to negated outputs;
    scaling a row leaves its normalisation unchanged.  Linear is x @ W
    (Burn's [d_in, d_out] weight layout), checked against numpy.matmul."""
    w = np.linspace(0.5, 1.5, 16).astype(np.float32)
    x = np.stack([np.full(16, 3.0), np.full(16, -0.25), np.full(16, 1e-5)]).astype(np.float32)
    out = oracle.rmsnorm(x, w)
    eps = 8.1584695e-8
    for r, c in enumerate((3.0, -0.25, 1e-5)):
        np.testing.assert_allclose(out[r], c / np.sqrt(c * c + eps) * w, rtol=1e-6)
    rng = np.random.default_rng(0)
    v = rng.standard_normal((2, 16)).astype(np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(-v, w), -oracle.rmsnorm(v, w), rtol=1e-6)
    np.testing.assert_allclose(oracle.rmsnorm(7 * v, w), oracle.rmsnorm(v, w), rtol=1e-5)
    X = rng.standard_normal((3, 5)).astype(np.float32)
    W = rng.standard_normal((5, 4)).astype(np.float32)
    bias = rng.standard_normal(4).astype(np.float32)
    np.testing.assert_allclose(oracle.linear(X, W), X.astype(np.float64) @ W, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.linear(X, W, bias), X.astype(np.float64) @ W + bias, rtol=1e-6, atol=1e-6)


def test_conv1d_step_unroll_equals_convolution():
    """Stepping the causal depthwise conv window token by token equals a full
    causal convolution (numpy.convolve) of the sequence prefixed by the initial
    window; plus bias and SiLU."""
    rng = np.random.default_rng(21)
    b, c, k, L = 2, 5, 4, 9
    w = rng.standard_normal((c, k)).astype(np.float32)
    bias = rng.standard_normal(c).astype(np.float32)
    st0 = rng.standard_normal((b, c, k)).astype(np.float32)
    xs = rng.standard_normal((L, b, c)).astype(np.float32)
    st = st0
    for t in range(L):
        out, st = oracle.conv1d_step(xs[t], st, w, bias, silu=(t % 2 == 0))
        for bi in range(b):
            for ci in range(c):
                seq = np.concatenate([st0[bi, ci], xs[:t + 1, bi, ci]]).astype(np.float64)
                full = np.convolve(seq, w[ci, ::-1].astype(np.float64), mode="valid")  # correlation
                v = full[t + 1] + bias[ci]
                ref = v / (1 + np.exp(-v)) if t % 2 == 0 else v
                np.testing.assert_allclose(out[bi, ci], ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(st[:, :, -1], xs[-1])


# ------------------------------------------------------------- Mamba-3 step --

def _mamba3_seq(seed, b, L, M, H, P, N):
    rng = np.random.default_rng(seed)
    dt = rng.uniform(0.01, 0.3, (b, L, H))
    A = -rng.uniform(0.5, 2.0, H)
    lam = 1.0 / (1.0 + np.exp(-rng.standard_normal((b, L, H))))
    da = dt * A
    alpha, beta, gamma = np.exp(da), (1 - lam) * dt * np.exp(da), lam * dt
    x = rng.standard_normal((b, L, H, P)).astype(np.float32)
    B = (rng.standard_normal((b, L, M, H, N)) / np.sqrt(N)).astype(np.float32)
    C = (rng.standard_normal((b, L, M, H, N)) / np.sqrt(N)).astype(np.float32)
    mimo_x = None if M == 1 else rng.standard_normal((H, M, P)).astype(np.float32)
    D = rng.standard_normal(H).astype(np.float32)
    return dict(dt=dt, lam=lam, da=da, alpha=alpha, beta=beta, gamma=gamma, x=x, B=B, C=C, mimo_x=mimo_x, D=D)


@pytest.mark.parametrize("M", [1, 4])
def test_mamba3_step_core_unroll_equals_chunked_ssd3(M):
    """Token steps from an empty cache (double-SSD recurrence, the beta term
    built from the previous token's B and x) equal the pinned chunked
    single-SSD forward with scale_t = gamma_t + (1 - lambda_{t+1}) dt_{t+1}
    (single_ssd/single_ssd/mod.rs:129-150), plus the D skip on v."""
    b, L, H, P, N = 2, 13, 2, 8, 8
    d = _mamba3_seq(3 + M, b, L, M, H, P, N)
    st = np.zeros((b, H, P, N), np.float32)
    K = np.zeros((b, M, H, N), np.float32)
    vs = np.zeros((b, H, P), np.float32)
    outs = []
    for t in range(L):
        o, st = oracle.mamba3_step_core(d["x"][:, t], vs, d["B"][:, t], K, d["C"][:, t], d["alpha"][:, t],
                                        d["beta"][:, t], d["gamma"][:, t], st, d["mimo_x"], d["D"])
        outs.append(o)
        K, vs = d["B"][:, t], d["x"][:, t]
    out = np.stack(outs, 1)  # [b, L, M, H, P]
    mx = np.ones((H, M, P), np.float32) if d["mimo_x"] is None else d["mimo_x"]
    v = d["x"][:, :, None] * mx.transpose(1, 0, 2)[None, None]  # [b, L, M, H, P]
    nxt = np.concatenate([(1 - d["lam"][:, 1:]) * d["dt"][:, 1:], np.zeros((b, 1, H))], 1)
    scale = (d["gamma"] + nxt).astype(np.float32)
    y, hT = oracle.ssd3(v, d["da"].astype(np.float32), d["B"], d["C"], d["gamma"].astype(np.float32), scale,
                        None, chunk=4)
    # the step's state round-trips through f32 between tokens (as the cache does)
    np.testing.assert_allclose(out, y + d["D"][None, None, None, :, None] * v, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(st, hT, rtol=1e-5, atol=1e-6)


def _mamba3_params(seed, H, P, G, N, M, rope_dim, rng=None):
    rng = rng or np.random.default_rng(seed)
    return dict(nheads=H, headdim=P, ngroups=G, dstate=N, mimo=M, rope_dim=rope_dim,
                dt_bias=rng.uniform(-3, -1, H).astype(np.float32), a_floor=1e-4, dt_limit=(0.0, 65504.0),
                rotation_range=2.0, b_norm_w=rng.uniform(0.5, 1.5, N).astype(np.float32),
                c_norm_w=rng.uniform(0.5, 1.5, N).astype(np.float32),
                b_bias=(0.1 * rng.standard_normal((H, M, N))).astype(np.float32),
                c_bias=(0.1 * rng.standard_normal((H, M, N))).astype(np.float32))


def _mamba3_proj(rng, b, p):
    H, P, G, N, M = (p[k] for k in ("nheads", "headdim", "ngroups", "dstate", "mimo"))
    A = oracle.mamba3_num_angles(p["rope_dim"])
    return rng.standard_normal((b, 2 * H * P + 2 * M * G * N + 3 * H + A)).astype(np.float32)


@pytest.mark.parametrize("M,rope_frac", [(1, 1.0), (4, 1.0), (1, 0.5), (4, 0.5)])
def test_mamba3_step_prep_rotation_closed_form(M, rope_frac):
    """The rotation equals a complex multiply by exp(i theta) on each pair
    ((2a, 2a+1) for M = 1, (a, a + N/2) otherwise, rope.rs:34-170), preserves
    norms, leaves the unrotated entries alone, and theta is the wrapped
    cumulative angle prev + dt range pi tanh(rot)."""
    H, P, G, N, b = 4, 8, 2, 16, 3
    rope_dim = int(N * rope_frac)
    p = _mamba3_params(5, H, P, G, N, M, rope_dim)
    rng = np.random.default_rng(7)
    proj = _mamba3_proj(rng, b, p)
    A = oracle.mamba3_num_angles(rope_dim)
    ang0 = rng.uniform(-3, 3, (b, H, A)).astype(np.float32)
    r = oracle.mamba3_step_prep(proj, p, ang0)
    p0 = dict(p, rope_dim=0)
    r0 = oracle.mamba3_step_prep(proj[:, :proj.shape[1] - A + 1] if A != 1 else proj, p0,
                                 np.zeros((b, H, 1), np.float32))  # unrotated B/C (rot channel ignored)
    rot = proj[:, -A:]
    inc = r["dt"][:, :, None] * np.tanh(rot)[:, None, :] * (2.0 * np.pi)
    theta = np.angle(np.exp(1j * (ang0 + inc)))
    # outputs are f32 arrays: f32-level tolerances
    np.testing.assert_allclose(np.cos(r["angle"]), np.cos(theta), atol=2e-6)
    np.testing.assert_allclose(np.sin(r["angle"]), np.sin(theta), atol=2e-6)
    assert np.all(np.abs(r["angle"]) <= np.pi + 1e-6)
    i0 = np.arange(rope_dim // 2) * (2 if M == 1 else 1)
    i1 = i0 + (1 if M == 1 else N // 2)
    for key in ("B", "C"):
        u, w = r0[key], r[key]
        z = (u[..., i0] + 1j * u[..., i1]) * np.exp(1j * r["angle"][:, None, :, :rope_dim // 2])
        np.testing.assert_allclose(w[..., i0], z.real, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(w[..., i1], z.imag, rtol=1e-6, atol=1e-6)
        rest = np.setdiff1d(np.arange(N), np.concatenate([i0, i1]))
        np.testing.assert_allclose(w[..., rest], u[..., rest], rtol=0, atol=0)


def test_mamba3_step_prep_coefficients_and_norm():
    """Trapezoid coefficients: beta/alpha + gamma = dt (the two endpoint
    weights share dt), lambda -> 1 gives beta -> 0, the a_floor clamp and the
    dt clamp; QK-norm: a constant raw row normalises to sign(c) w (+ bias)."""
    H, P, G, N, M, b = 2, 4, 1, 8, 2, 2
    p = _mamba3_params(9, H, P, G, N, M, 0)
    rng = np.random.default_rng(11)
    proj = _mamba3_proj(rng, b, p)
    d_inner, bc = H * P, M * G * N
    o_dt, o_a, o_l = 2 * d_inner + 2 * bc, 2 * d_inner + 2 * bc + H, 2 * d_inner + 2 * bc + 2 * H
    r = oracle.mamba3_step_prep(proj, p, np.zeros((b, H, 1), np.float32))
    np.testing.assert_allclose(r["beta"] / r["alpha"] + r["gamma"], r["dt"], rtol=1e-6)
    softplus = lambda v: np.log1p(np.exp(v))  # noqa: E731
    dt = softplus(proj[:, o_dt:o_dt + H] + p["dt_bias"])
    np.testing.assert_allclose(r["dt"], dt, rtol=1e-6)
    a = -np.maximum(softplus(proj[:, o_a:o_a + H]), p["a_floor"])
    np.testing.assert_allclose(r["alpha"], np.exp(dt * a), rtol=1e-6)
    pr = proj.copy()
    pr[:, o_l:o_l + H] = 40.0          # lambda -> 1
    pr[:, o_a:o_a + H] = -60.0         # softplus below a_floor
    pr[:, 2 * d_inner:2 * d_inner + bc] = -2.5  # constant B rows
    r2 = oracle.mamba3_step_prep(pr, dict(p, dt_limit=(0.0, 0.05)), np.zeros((b, H, 1), np.float32))
    assert np.all(r2["beta"] < 1e-17) and np.all(r2["dt"] <= 0.05)
    np.testing.assert_allclose(r2["alpha"], np.exp(-r2["dt"] * p["a_floor"]), rtol=1e-6)
    want = -p["b_norm_w"][None, None, None, :] / np.sqrt(1 + 8.1584695e-8 / 6.25) + p["b_bias"].transpose(1, 0, 2)[None]
    np.testing.assert_allclose(r2["B"], np.broadcast_to(want, r2["B"].shape), rtol=1e-7)


def test_mamba3_step_finish_known_answers():
    """z = 0 closes the gate; a one-hot mimo_o selects one rank; the gated
    norm of a constant row is sign(c) w silu(z)."""
    rng = np.random.default_rng(13)
    b, M, H, P = 2, 3, 2, 4
    out = rng.standard_normal((b, M, H, P)).astype(np.float32)
    z = rng.standard_normal((b, H * P)).astype(np.float32)
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    y1 = oracle.mamba3_step_finish(out[:, :1], np.zeros_like(z))
    np.testing.assert_array_equal(y1, 0)
    mo = np.zeros((H, M, P), np.float32)
    mo[:, 1] = 1.0
    y = oracle.mamba3_step_finish(out, z, np.ones((H, M, P), np.float32), mo)
    np.testing.assert_allclose(y, (out[:, 1] * silu(z.reshape(b, H, P))).reshape(b, -1), rtol=1e-6)
    const = np.full((b, 1, H, P), -0.7, np.float32)
    w = rng.uniform(0.5, 1.5, P).astype(np.float32)
    yn = oracle.mamba3_step_finish(const, z, norm_w=w)
    want = -w[None, None] / np.sqrt(1 + 8.1584695e-8 / 0.49) * silu(z.reshape(b, H, P))
    np.testing.assert_allclose(yn, want.reshape(b, -1), rtol=1e-7)


def test_mamba3_prep_fwd_equals_step_prep():
    """The prefill prep over a sequence equals the pinned per-token prep run
    token by token (angles compared on the circle), and its cache tail is the
    last token's."""
    H, P, G, N, M, b, s = 4, 8, 2, 16, 4, 2, 9
    p = _mamba3_params(41, H, P, G, N, M, 16)
    p.update(mimo_x=np.random.default_rng(1).standard_normal((H, M, P)).astype(np.float32))
    rng = np.random.default_rng(43)
    A = oracle.mamba3_num_angles(16)
    proj = np.stack([_mamba3_proj(rng, b, p) for _ in range(s)], 1)
    cache = dict(ssm=np.zeros((b, H, P, N), np.float32), k_state=np.zeros((b, M, H, N), np.float32),
                 v_state=np.zeros((b, H, P), np.float32), angle=rng.uniform(-3, 3, (b, H, A)).astype(np.float32))
    r = oracle.mamba3_prep_fwd(proj, p, cache)
    ang = cache["angle"]
    for t in range(s):
        st = oracle.mamba3_step_prep(proj[:, t], p, ang)
        ang = st["angle"]
        np.testing.assert_allclose(r["B"][:, t], st["B"], rtol=2e-5, atol=2e-6)
        np.testing.assert_allclose(r["C"][:, t], st["C"], rtol=2e-5, atol=2e-6)
        np.testing.assert_allclose(r["gamma"][:, t], st["gamma"], rtol=1e-6)
        np.testing.assert_allclose(np.exp(r["da"][:, t]), st["alpha"], rtol=1e-6)
    np.testing.assert_allclose(np.cos(r["angle"]), np.cos(ang), atol=2e-6)
    np.testing.assert_allclose(np.sin(r["angle"]), np.sin(ang), atol=2e-6)
    np.testing.assert_allclose(r["k_state"], r["B"][:, -1])


@pytest.mark.parametrize("M,out_norm", [(1, False), (4, True)])
def test_mamba3_prefill_then_steps_equals_steps(M, out_norm):
    """A prefill (prep -> pinned chunked SSD -> finish) of the first s1 tokens,
    then per-token steps from its cache, equals per-token steps from an empty
    cache for every token (the reference's split-prefill/step parity,
    single_ssd/single_ssd/tests.rs) -- this pins the beta seed, scale and the
    cache handover."""
    H, P, G, N, b, s1, s2 = 2, 8, 1, 16, 2, 7, 3
    p = _mamba3_params(47 + M, H, P, G, N, M, 16)
    rng = np.random.default_rng(53)
    if M > 1:
        p.update(mimo_x=rng.standard_normal((H, M, P)).astype(np.float32),
                 mimo_z=rng.standard_normal((H, M, P)).astype(np.float32),
                 mimo_o=rng.standard_normal((H, M, P)).astype(np.float32))
    if out_norm:
        p.update(out_norm_w=rng.uniform(0.5, 1.5, P).astype(np.float32))
    p.update(D=rng.standard_normal(H).astype(np.float32))
    A = oracle.mamba3_num_angles(16)
    proj = np.stack([_mamba3_proj(rng, b, p) for _ in range(s1 + s2)], 1)
    zero = dict(ssm=np.zeros((b, H, P, N), np.float32), k_state=np.zeros((b, M, H, N), np.float32),
                v_state=np.zeros((b, H, P), np.float32), angle=np.zeros((b, H, A), np.float32))
    # reference: token steps from the empty cache
    ys, c = [], zero
    for t in range(s1 + s2):
        y, c = oracle.mamba3_step(proj[:, t], p, c)
        ys.append(y)
    # prefill of the first s1 tokens
    r = oracle.mamba3_prep_fwd(proj[:, :s1], p, zero)
    yssd, hT = oracle.ssd3(r["v"], r["da"], r["B"], r["C"], r["gamma"], r["scale"], r["h0"], chunk=4)
    d_inner = H * P
    yp = oracle.mamba3_finish_fwd(yssd, r["v"], proj[:, :s1, :d_inner], p)
    for t in range(s1):
        np.testing.assert_allclose(yp[:, t], ys[t], rtol=2e-4, atol=2e-5)
    c = dict(ssm=hT, k_state=r["k_state"], v_state=r["v_state"], angle=r["angle"])
    for t in range(s1, s1 + s2):
        y, c = oracle.mamba3_step(proj[:, t], p, c)
        np.testing.assert_allclose(y, ys[t], rtol=2e-4, atol=2e-5)


# ---------------------------------------------------------- Mamba-2 block forward --

@pytest.mark.parametrize("K,L", [(4, 9), (4, 2), (1, 5), (3, 3)])
def test_mamba2_conv_fwd_equals_conv_steps(K, L):
    """The prefill conv (mamba2.rs:618-699) over L tokens equals L single conv
    steps of the C oracle (conv1d_step, the decode window of mamba2.rs:870-905)
    from the same cache, outputs and final window (also when L < K)."""
    rng = np.random.default_rng(K * 10 + L)
    b, c = 2, 12
    proj = rng.standard_normal((b, L, c + 9)).astype(np.float32)
    w = rng.standard_normal((c, K)).astype(np.float32)
    bias = rng.standard_normal(c).astype(np.float32)
    st = rng.standard_normal((b, c, K)).astype(np.float32)
    xbc, _, ns = oracle.mamba2_conv_fwd(proj, w, bias, st, np.zeros(3, np.float32), 4, 4 + c, c, 3)
    s = st.copy()
    for l in range(L):
        o, s = oracle.conv1d_step(proj[:, l, 4:4 + c], s, w, bias, True)
        np.testing.assert_allclose(xbc[:, l], o, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ns, s, rtol=0, atol=0)


def test_mamba2_conv_fwd_dt_closed_form():
    """dt = clamp(softplus(raw + bias)): log(2) at zero, the identity above the
    threshold, and the clamp limits."""
    proj = np.array([[[0.0, 30.0, -40.0]]], np.float32)
    _, dt, _ = oracle.mamba2_conv_fwd(proj, np.ones((1, 1), np.float32), None, np.zeros((1, 1, 1), np.float32),
                                      np.zeros(3, np.float32), 0, 0, 1, 3, dt_limit=(1e-3, 25.0))
    np.testing.assert_allclose(dt[0, 0], [np.log(2.0), 25.0, 1e-3], rtol=1e-12)


def test_mamba2_gated_rmsnorm_closed_forms():
    """A constant row normalises to sign * gamma (up to eps); the norm is scale
    invariant; norm-then-gate multiplies the normalised row by silu(z)."""
    W = 16
    gamma = np.linspace(0.5, 1.5, W)
    z = np.full((1, W), 0.7)
    y = np.full((1, W), -3.0)
    out = oracle.mamba2_gated_rmsnorm(y, z, gamma, 1e-12)
    np.testing.assert_allclose(out[0], -gamma, rtol=1e-9)
    rng = np.random.default_rng(3)
    y2, z2 = rng.standard_normal((4, W)), rng.standard_normal((4, W))
    np.testing.assert_allclose(oracle.mamba2_gated_rmsnorm(5.0 * y2, z2, gamma, 1e-14),
                               oracle.mamba2_gated_rmsnorm(y2, z2, gamma, 1e-14), rtol=1e-9)
    sz = 0.7 / (1 + np.exp(-0.7))
    np.testing.assert_allclose(oracle.mamba2_gated_rmsnorm(y, z, gamma, 1e-12, norm_before_gate=True)[0],
                               -gamma * sz, rtol=1e-9)


@pytest.mark.parametrize("norm_before_gate", [False, True])
def test_mamba2_block_fwd_equals_steps(norm_before_gate):
    """Mamba2::forward between the projections over L tokens (conv prologue ->
    SSD -> gated norm) equals L decode steps (the C oracle's mamba2_step_ssm,
    pinned against its own closed forms) from the same caches: every token's
    output and both final caches."""
    rng = np.random.default_rng(11 + norm_before_gate)
    b, L, H, P, G, N, K = 2, 10, 4, 8, 2, 8, 4
    d_inner = H * P
    conv_dim = d_inner + 2 * G * N
    row = d_inner + conv_dim + H
    cfg = dict(nheads=H, headdim=P, ngroups=G, dstate=N, norm_before_gate=norm_before_gate)
    p = dict(conv_w=(rng.standard_normal((conv_dim, K)) / 2).astype(np.float32),
             conv_b=(0.1 * rng.standard_normal(conv_dim)).astype(np.float32),
             dt_bias=rng.uniform(-3, -1, H).astype(np.float32),
             A=(-np.exp(rng.uniform(0, np.log(8), H))).astype(np.float32),
             D=rng.standard_normal(H).astype(np.float32), norm_w=rng.uniform(0.5, 1.5, d_inner).astype(np.float32))
    proj = rng.standard_normal((b, L, row)).astype(np.float32)
    cs0 = rng.standard_normal((b, conv_dim, K)).astype(np.float32)
    ss0 = (0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32)
    y, cs, ss = oracle.mamba2_block_fwd(proj, p, cs0, ss0, chunk=4, cfg=cfg)
    c_s, s_s = cs0, ss0
    for l in range(L):
        o, c_s, s_s = oracle.mamba2_step_ssm(proj[:, l], c_s, p["conv_w"], p["conv_b"], p["dt_bias"], p["A"], p["D"],
                                             p["norm_w"], s_s, H, P, G, N, norm_before_gate=norm_before_gate)
        np.testing.assert_allclose(y[:, l], o, rtol=2e-4, atol=2e-5)
    np.testing.assert_allclose(cs, c_s, rtol=0, atol=0)
    np.testing.assert_allclose(ss, s_s, rtol=1e-4, atol=1e-6)


# ---------------------------------------------------------------------------
# Mamba-1 block forward (src/mamba1/mamba1.rs:278-352) against the block step
# unrolled token by token, and prefix + suffix forward against one forward:
# the reference's own relations (src/mamba1/mamba1/tests.rs:216-372, 384-429)
# ---------------------------------------------------------------------------

def _m1_params(seed, d_model, n, k, expand, dt_rank=None):
    """Random Mamba-1 parameters with the reference init's scales
    (src/mamba1/mamba1.rs:124-227); Linear weights [d_in, d_out]."""
    rng = np.random.default_rng(seed)
    di = expand * d_model
    r = dt_rank or -(-d_model // n)

    def uni(shape, bound):
        return ((rng.random(shape) * 2 - 1) * bound).astype(np.float32)

    dt = np.exp(rng.random(di) * (np.log(0.1) - np.log(1e-3)) + np.log(1e-3))
    return dict(in_proj_w=uni((d_model, 2 * di), d_model ** -0.5), conv_w=uni((di, k), k ** -0.5),
                conv_b=uni((di,), k ** -0.5), x_proj_w=uni((di, r + 2 * n), di ** -0.5),
                dt_proj_w=uni((r, di), r ** -0.5), dt_proj_b=(dt + np.log(-np.expm1(-dt))).astype(np.float32),
                A=-np.tile(np.arange(1, n + 1, dtype=np.float32), (di, 1)), D=np.ones(di, np.float32),
                out_proj_w=uni((di, d_model), di ** -0.5))


def _m1_cache(seed, b, di, k, n, random):
    rng = np.random.default_rng(seed)
    if not random:
        return np.zeros((b, di, k), np.float32), np.zeros((b, di, n), np.float32)
    return (rng.standard_normal((b, di, k)).astype(np.float32),
            rng.standard_normal((b, di, n)).astype(np.float32))


# (d_model, state_rank, conv_kernel, expand, dt_rank): the reference's small
# config and its d_state 16, d_conv 2, expand 1 and custom dt_rank variants
M1_CFGS = [(32, 8, 4, 2, None), (32, 16, 4, 2, None), (32, 8, 2, 2, None), (32, 8, 4, 1, None), (32, 8, 4, 2, 8)]


@pytest.mark.parametrize("cfg", M1_CFGS)
@pytest.mark.parametrize("random_init", [False, True])
def test_mamba1_block_forward_equals_step_unroll(cfg, random_init):
    dm, n, k, ex, r = cfg
    p = _m1_params(1, dm, n, k, ex, r)
    b, L = 2, 5
    x = np.random.default_rng(2).standard_normal((b, L, dm)).astype(np.float32)
    conv0, ssm0 = _m1_cache(3, b, ex * dm, k, n, random_init)
    y, conv, ssm = oracle.mamba1_block_fwd(x, p, conv0, ssm0)
    cs, ss, ys = conv0, ssm0, []
    for t in range(L):
        yt, cs, ss = oracle.mamba1_block_step(np.ascontiguousarray(x[:, t]), p, cs, ss)
        ys.append(yt)
    np.testing.assert_allclose(y, np.stack(ys, 1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(conv, cs, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(ssm, ss, rtol=1e-5, atol=1e-6)
    if random_init:
        # the initial state is consumed: a zero cache gives a clearly different output
        y0, _, _ = oracle.mamba1_block_fwd(x, p, *_m1_cache(3, b, ex * dm, k, n, False))
        assert np.abs(y - y0).max() > 1e-3


def test_mamba1_block_split_equals_full():
    dm, n, k, ex, r = M1_CFGS[0]
    p = _m1_params(4, dm, n, k, ex, r)
    b, L, split = 2, 6, 2
    x = np.random.default_rng(5).standard_normal((b, L, dm)).astype(np.float32)
    conv0, ssm0 = _m1_cache(6, b, ex * dm, k, n, True)
    y, conv, ssm = oracle.mamba1_block_fwd(x, p, conv0, ssm0)
    ya, ca, sa = oracle.mamba1_block_fwd(x[:, :split], p, conv0, ssm0)
    yb, cb, sb = oracle.mamba1_block_fwd(x[:, split:], p, ca, sa)
    np.testing.assert_allclose(y, np.concatenate([ya, yb], 1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(conv, cb, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(ssm, sb, rtol=1e-5, atol=1e-6)


def test_mamba1_block_forward_short_sequence_window():
    """A sequence shorter than the conv kernel: the new window keeps the old
    window's tail (mamba1.rs:317-325), checked by hand against the padded input."""
    dm, n, k, ex, r = 16, 4, 4, 2, None
    p = _m1_params(7, dm, n, k, ex, r)
    b, L = 1, 2
    x = np.random.default_rng(8).standard_normal((b, L, dm)).astype(np.float32)
    conv0, ssm0 = _m1_cache(9, b, ex * dm, k, n, True)
    _, conv, _ = oracle.mamba1_block_fwd(x, p, conv0, ssm0)
    xs = oracle.linear(x.reshape(b * L, dm), p["in_proj_w"])[:, :ex * dm].reshape(b, L, ex * dm)
    pad = np.concatenate([conv0[:, :, 1:], xs.transpose(0, 2, 1)], axis=2)
    np.testing.assert_allclose(conv, pad[:, :, L - 1:L - 1 + k], rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------------
# Mamba-2 SSD backward (oracle.ssd2_bwd): pinned by finite differences of an
# independent float64 forward in the segsum (matrix) form, itself tied to
# oracle.ssd2, and by closed forms.
# --------------------------------------------------------------------------

def _ssd2_fwd64(x, dt, A, B, C, D, h0):
    """Whole-sequence segsum form (ssd_minimal with one chunk, minimal.rs:95-496)
    in float64: y = (L o C B^T)(dt x) + exp(cs) C h0^T + D x, h_L from the same
    weights.  Independent of the recurrence the backward oracle runs."""
    b, l, h, p = x.shape
    g = B.shape[2]
    rep = h // g
    Bh, Ch = np.repeat(B, rep, axis=2), np.repeat(C, rep, axis=2)
    cs = np.cumsum(dt * A[None, None, :], axis=1)                     # [b, l, h]
    seg = cs[:, :, None, :] - cs[:, None, :, :]                      # [b, t, s, h]
    tri = np.tril(np.ones((l, l), bool))[None, :, :, None]
    Lm = np.where(tri, np.exp(np.where(tri, seg, 0.0)), 0.0)
    CB = np.einsum("bthn,bshn->btsh", Ch, Bh)
    y = np.einsum("btsh,bsh,bshp->bthp", Lm * CB, dt, x)
    y += np.exp(cs)[..., None] * np.einsum("bthn,bhpn->bthp", Ch, h0)
    y += D[None, None, :, None] * x
    wend = np.exp(cs[:, -1:, :] - cs) * dt                            # [b, s, h]
    hT = np.exp(cs[:, -1])[:, :, None, None] * h0 + np.einsum("bsh,bshp,bshn->bhpn", wend, x, Bh)
    return y, hT


def _ssd2_bwd_case(seed, b=1, l=6, h=2, p=3, g=1, n=4):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s)  # noqa: E731
    return dict(x=r(b, l, h, p), dt=rng.uniform(0.05, 0.6, (b, l, h)), A=-rng.uniform(0.3, 2.0, h),
                B=r(b, l, g, n), C=r(b, l, g, n), D=r(h), h0=r(b, h, p, n)), r(b, l, h, p), r(b, h, p, n)


def test_ssd2_fwd64_matches_oracle_forward():
    """The float64 matrix form used for the finite differences equals oracle.ssd2."""
    inp, _, _ = _ssd2_bwd_case(3, b=2, l=9, h=4, p=5, g=2, n=6)
    y, hT = _ssd2_fwd64(**inp)
    yo, ho = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"], form="recurrent")
    np.testing.assert_allclose(y, yo, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(hT, ho, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("g", [1, 2])
def test_ssd2_bwd_equals_finite_differences(g):
    """Every gradient of oracle.ssd2_bwd equals the central difference of
    L = sum dy.y + sum dfinal.h_L through the float64 forward, at every
    coordinate (tiny shapes; dB/dC in group form sum the group's heads)."""
    inp, dy, dF = _ssd2_bwd_case(11 + g, b=2, l=5, h=2, p=3, g=g, n=4)
    grads = oracle.ssd2_bwd(dy, dF, **inp)

    def loss(a):
        y, hT = _ssd2_fwd64(**a)
        return float((y * dy).sum() + (hT * dF).sum())
    eps = 1e-6
    names = dict(x="dx", dt="ddt", A="dA", B="dB", C="dC", D="dD", h0="dh0")
    for k, gk in names.items():
        fd = np.zeros_like(inp[k])
        for idx in np.ndindex(inp[k].shape):
            a = {kk: vv.copy() for kk, vv in inp.items()}
            a[k][idx] += eps
            lp = loss(a)
            a[k][idx] -= 2 * eps
            fd[idx] = (lp - loss(a)) / (2 * eps)
        np.testing.assert_allclose(grads[gk], fd, rtol=1e-6, atol=1e-7, err_msg=k)


def test_ssd2_bwd_closed_forms():
    """With dy = 0 only the final state carries gradient: dh0 = exp(A sum dt)
    dfinal and dC = 0; dD = sum x.dy for any dy."""
    inp, dy, dF = _ssd2_bwd_case(21, b=2, l=7, h=3, p=2, g=1, n=3)
    gz = oracle.ssd2_bwd(np.zeros_like(dy), dF, **inp)
    decay = np.exp(inp["A"][None, :] * inp["dt"].sum(1))              # [b, h]
    np.testing.assert_allclose(gz["dh0"], decay[:, :, None, None] * dF, rtol=1e-12)
    np.testing.assert_allclose(gz["dC"], 0.0, atol=0)
    gd = oracle.ssd2_bwd(dy, None, **inp)
    np.testing.assert_allclose(gd["dD"], np.einsum("blhp,blhp->h", inp["x"], dy), rtol=1e-12)


def _ssd3_fwd64(v, da, B, C, gamma, scale, h0):
    """Whole-sequence matrix form of the Mamba-3 single-SSD forward in float64
    (the fused-axis K5 of single_ssd/ssd/serial.rs:56-268 with one chunk): y =
    (W o C B^T) v + exp(cs) C h0^T with W = exp(cs_t - cs_s) scale_s for s < t
    and gamma_t for s = t; h_L from the same weights.  gamma / scale None = 1.
    Group-form B / C [b, l, m, g, n].  Independent of the backward oracle's
    recurrence."""
    b, l, m, h, p = v.shape
    g = B.shape[3]
    rep = h // g
    Bh, Ch = np.repeat(B, rep, axis=3), np.repeat(C, rep, axis=3)
    gam = np.ones((b, l, h)) if gamma is None else gamma
    scl = np.ones((b, l, h)) if scale is None else scale
    cs = np.cumsum(da, axis=1)                                         # [b, l, h]
    seg = cs[:, :, None, :] - cs[:, None, :, :]                        # [b, t, s, h]
    lower = np.tril(np.ones((l, l), bool), -1)[None, :, :, None]
    eye = np.eye(l, dtype=bool)[None, :, :, None]
    W = np.where(lower, np.exp(np.where(lower, seg, 0.0)) * scl[:, None, :, :], 0.0)
    W = W + np.where(eye, gam[:, :, None, :], 0.0)
    y = np.einsum("btsh,btohn,bsihn,bsihp->btohp", W, Ch, Bh, v)
    y += np.exp(cs)[:, :, None, :, None] * np.einsum("btohn,bhpn->btohp", Ch, h0)
    wend = np.exp(cs[:, -1:, :] - cs) * scl                            # [b, s, h]
    hT = np.exp(cs[:, -1])[:, :, None, None] * h0 + np.einsum("bsh,bsihp,bsihn->bhpn", wend, v, Bh)
    return y, hT


def _ssd3_bwd_case(seed, b=2, l=4, m=2, h=2, p=2, g=1, n=3, weights=True):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s)  # noqa: E731
    inp = dict(v=r(b, l, m, h, p), da=-rng.uniform(0.05, 0.8, (b, l, h)), B=r(b, l, m, g, n), C=r(b, l, m, g, n),
               gamma=rng.uniform(0.05, 0.6, (b, l, h)) if weights else None,
               scale=rng.uniform(0.1, 0.9, (b, l, h)) if weights else None, h0=r(b, h, p, n))
    return inp, r(b, l, m, h, p), r(b, h, p, n)


def test_ssd3_fwd64_matches_oracle_forward():
    """The float64 matrix form used for the finite differences equals the C
    oracle's single-SSD forward (per-head B / C, f32-representable inputs)."""
    inp, _, _ = _ssd3_bwd_case(5, b=2, l=9, m=3, h=2, p=4, g=2, n=5)
    inp = {k: v.astype(np.float32).astype(np.float64) for k, v in inp.items()}
    y, hT = _ssd3_fwd64(**inp)
    yo, ho = oracle.ssd3(inp["v"], inp["da"], inp["B"], inp["C"], inp["gamma"], inp["scale"], inp["h0"], chunk=4)
    np.testing.assert_allclose(y, yo, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(hT, ho, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("g,weights", [(1, True), (2, True), (1, False)])
def test_ssd3_bwd_equals_finite_differences(g, weights):
    """Every gradient of oracle.ssd3_bwd equals the central difference of
    L = sum dy.y + sum dfinal.h_L through the float64 forward at every
    coordinate: the single seam (gamma, scale given) and the double seam
    (unit weights); dB / dC in group form sum the group's heads."""
    inp, dy, dF = _ssd3_bwd_case(31 + g + 2 * weights, g=g, weights=weights)
    grads = oracle.ssd3_bwd(dy, dF, **inp)

    def loss(a):
        y, hT = _ssd3_fwd64(**a)
        return float((y * dy).sum() + (hT * dF).sum())
    eps = 1e-6
    names = dict(v="dv", da="dda", B="dB", C="dC", h0="dh0")
    if weights:
        names.update(gamma="dgamma", scale="dscale")
    else:
        assert grads["dgamma"] is None and grads["dscale"] is None
    for k, gk in names.items():
        fd = np.zeros_like(inp[k])
        for idx in np.ndindex(inp[k].shape):
            a = {kk: (None if vv is None else vv.copy()) for kk, vv in inp.items()}
            a[k][idx] += eps
            lp = loss(a)
            a[k][idx] -= 2 * eps
            fd[idx] = (lp - loss(a)) / (2 * eps)
        np.testing.assert_allclose(grads[gk], fd, rtol=1e-6, atol=1e-7, err_msg=k)


def test_ssd3_bwd_reduces_to_mamba2():
    """MIMO rank 1 with v = x, da = dt A, scale = gamma = dt is the Mamba-2 SSD
    (no D): the gradients equal oracle.ssd2_bwd's, with ddt = A dda + dscale +
    dgamma and dA = sum dt dda."""
    inp, dy, dF = _ssd2_bwd_case(41, b=2, l=6, h=4, p=3, g=2, n=5)
    x, dt, A = inp["x"], inp["dt"], inp["A"]
    g2 = oracle.ssd2_bwd(dy, dF, x, dt, A, inp["B"], inp["C"], None, inp["h0"])
    g3 = oracle.ssd3_bwd(dy[:, :, None], dF, x[:, :, None], dt * A[None, None, :], inp["B"][:, :, None],
                         inp["C"][:, :, None], dt, dt, inp["h0"])
    np.testing.assert_allclose(g3["dv"][:, :, 0], g2["dx"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(g3["dB"][:, :, 0], g2["dB"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(g3["dC"][:, :, 0], g2["dC"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(g3["dh0"], g2["dh0"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(A[None, None, :] * g3["dda"] + g3["dscale"] + g3["dgamma"], g2["ddt"],
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose((dt * g3["dda"]).sum((0, 1)), g2["dA"], rtol=1e-12, atol=1e-12)


def test_ssd3_bwd_closed_forms():
    """With dy = 0 only the final state carries gradient: dh0 = exp(sum da)
    dfinal, dC = 0 and dgamma = 0."""
    inp, dy, dF = _ssd3_bwd_case(51, b=2, l=5, m=2, h=3, p=2, g=1, n=3)
    gz = oracle.ssd3_bwd(np.zeros_like(dy), dF, **inp)
    decay = np.exp(inp["da"].sum(1))                                    # [b, h]
    np.testing.assert_allclose(gz["dh0"], decay[:, :, None, None] * dF, rtol=1e-12)
    np.testing.assert_allclose(gz["dC"], 0.0, atol=0)
    np.testing.assert_allclose(gz["dgamma"], 0.0, atol=0)

