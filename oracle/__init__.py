"""CPU oracle for the burn-mamba SSM hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product path (``burn-mamba_amd/``) never imports it.

``liboracle.so`` (built from ``oracle_body.h`` by ``oracle/Makefile``) holds the
C restatement of the reference algorithms at two precisions: ``prec=32`` runs
every intermediate in f32 like the reference's f32 Burn ops, ``prec=64`` in f64
("truth").  Each wrapper below names the reference function it restates; the
exact file:line citations are in ``oracle_body.h``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        for prec in (32, 64):
            for name in ("ssd2_serial", "ssd2_minimal", "ssd2_recurrent", "mamba1_scan",
                         "mamba1_step", "mamba2_step_ssm", "rmsnorm", "linear", "ssd3_serial", "conv1d_step",
                         "ssd3_recurrent"):
                getattr(_lib, f"orc{prec}_{name}").restype = None
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _fn(name, prec):
    return getattr(lib(), f"orc{prec}_{name}")


# --------------------------------------------------------------------------
# Mamba-2 SSD core (src/mamba2/ssd/{serial,minimal}.rs; mamba2.rs:932-991)
# --------------------------------------------------------------------------

def ssd2(x, dt, A, B, C, D=None, h0=None, init_hpr=None, chunk=64, form="serial", prec=64):
    """Mamba-2 SSD forward. x[b,l,h,p] dt[b,l,h] A[h] B,C[b,l,g,n] D[h] h0[b,h,p,n].

    form: "serial" (K1..K5, serial.rs), "minimal" (segsum, minimal.rs) or
    "recurrent" (token-by-token step recurrence, mamba2.rs:932-991).
    Returns (y[b,l,h,p], final_state[b,h,p,n]) as float32.
    """
    x, dt, A, B, C, D, h0, init_hpr = map(_f32, (x, dt, A, B, C, D, h0, init_hpr))
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    assert dt.shape == (b, l, h) and A.shape == (h,) and B.shape == C.shape == (b, l, g, n)
    assert h % g == 0
    y = np.zeros_like(x)
    hT = np.zeros((b, h, p, n), np.float32)
    args = [_ptr(x), _ptr(dt), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(h0), _ptr(init_hpr),
            _ptr(y), _ptr(hT)]
    if form == "recurrent":
        _fn("ssd2_recurrent", prec)(b, l, h, p, g, n, *args)
    else:
        _fn(f"ssd2_{form}", prec)(b, l, h, p, g, n, chunk, *args)
    return y, hT


def ssd2_bwd(dy, dfinal, x, dt, A, B, C, D=None, h0=None):
    """Gradients of the Mamba-2 SSD forward (oracle.ssd2) in float64 numpy, by
    the per-token reverse recurrence: the analytic backward of
    Mamba2BackendExt::ssd_serial_recalculated that
    src/mamba2/ssd/serial_recalculated/combined_backward.rs:126-593 computes
    chunk-wise (its Autodiff arm, backward.rs:29-321), here token by token.

    Forward per (b, head): h_t = exp(dt_t A) h_{t-1} + dt_t x_t B_t^T,
    y_t = h_t C_t + D x_t, final state h_L.  With L = sum dy.y + sum dfinal.h_L
    and G_t = dL/dh_t (G_L = dfinal + dy_L C_L^T, G_{t-1} = exp(dt_t A) G_t +
    dy_{t-1} C_{t-1}^T):
      dC_t = h_t^T dy_t, dx_t = D dy_t + dt_t G_t B_t, dB_t = dt_t G_t^T x_t,
      d(dt_t A) = exp(dt_t A) <G_t, h_{t-1}>, ddt_t = A d(dt_t A) + x_t^T G_t B_t,
      dA = sum_t dt_t d(dt_t A), dD = sum_t x_t . dy_t, dh0 = exp(dt_1 A) G_1.
    x, dy [b,l,h,p]; dt [b,l,h]; A [h]; B, C [b,l,g,n] (group form, dB / dC
    summed over the group's heads); D [h] or None; h0 [b,h,p,n] or None;
    dfinal [b,h,p,n] or None.  Returns a dict of float64 gradients."""
    f = lambda t: None if t is None else np.asarray(t, np.float64)  # noqa: E731
    dy, dfinal, x, dt, A, B, C, D, h0 = map(f, (dy, dfinal, x, dt, A, B, C, D, h0))
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    rep = h // g
    Bh = np.repeat(B, rep, axis=2)   # [b, l, h, n]
    Ch = np.repeat(C, rep, axis=2)
    Dv = np.zeros(h) if D is None else D
    da = dt * A[None, None, :]       # [b, l, h]
    hs = np.zeros((l + 1, b, h, p, n))
    hs[0] = 0.0 if h0 is None else h0
    for t in range(l):
        hs[t + 1] = np.exp(da[:, t])[:, :, None, None] * hs[t] + \
            (dt[:, t][:, :, None] * x[:, t])[..., None] * Bh[:, t][:, :, None, :]
    G = np.zeros((b, h, p, n)) if dfinal is None else dfinal.copy()
    dx = np.zeros_like(x)
    ddt = np.zeros_like(dt)
    dBh = np.zeros_like(Bh)
    dCh = np.zeros_like(Ch)
    dA = np.zeros(h)
    for t in range(l - 1, -1, -1):
        G = G + dy[:, t][..., None] * Ch[:, t][:, :, None, :]
        dCh[:, t] = np.einsum("bhpn,bhp->bhn", hs[t + 1], dy[:, t])
        GB = np.einsum("bhpn,bhn->bhp", G, Bh[:, t])
        dx[:, t] = Dv[None, :, None] * dy[:, t] + dt[:, t][..., None] * GB
        dBh[:, t] = dt[:, t][..., None] * np.einsum("bhpn,bhp->bhn", G, x[:, t])
        dda = np.exp(da[:, t]) * np.einsum("bhpn,bhpn->bh", G, hs[t])
        xGB = np.einsum("bhp,bhp->bh", x[:, t], GB)
        ddt[:, t] = A[None, :] * dda + xGB
        dA += (dt[:, t] * dda).sum(0)
        G = np.exp(da[:, t])[:, :, None, None] * G
    dD = np.einsum("blhp,blhp->h", x, dy)
    return dict(dx=dx, ddt=ddt, dA=dA, dB=dBh.reshape(b, l, g, rep, n).sum(3),
                dC=dCh.reshape(b, l, g, rep, n).sum(3), dD=dD, dh0=G)


def ssd3_bwd(dy, dfinal, v, da, B, C, gamma=None, scale=None, h0=None):
    """Gradients of the Mamba-3 single-SSD forward (oracle.ssd3) in float64
    numpy by the per-token reverse recurrence: the analytic backward that
    src/mamba3/single_ssd/ssd/serial_recalculated/combined_backward.rs:74-536
    computes chunk-wise (its Autodiff arm, single_ssd/ssd/serial_recalculated/
    backward.rs:27-299), here token by token.  With gamma = scale = None (both
    1) it is the double-SSD seam's backward (double_ssd/ssd/serial_recalculated/
    combined_backward.rs:98-542, backward.rs:27-275), whose forward is the
    single one with unit weights.

    Forward per (b, head), K_t = sum_m v[t,m] B[t,m]^T (P x N):
      S_t = exp(da_t) h_{t-1},  h_t = S_t + scale_t K_t,
      y[t,mo] = S_t C[t,mo] + gamma_t sum_mi (C[t,mo].B[t,mi]) v[t,mi],
    final state h_L.  With G_t = dL/dh_t (G_L = dfinal) and
    Q_t = sum_mo dy[t,mo] C[t,mo]^T:
      dC[t,mo] = S_t^T dy[t,mo] + gamma_t sum_mi (dy[t,mo].v[t,mi]) B[t,mi]
      dB[t,mi] = scale_t G_t^T v[t,mi] + gamma_t sum_mo (dy[t,mo].v[t,mi]) C[t,mo]
      dv[t,mi] = scale_t G_t B[t,mi] + gamma_t sum_mo (C[t,mo].B[t,mi]) dy[t,mo]
      dscale_t = sum_mi v[t,mi]^T G_t B[t,mi]
      dgamma_t = sum_{mo,mi} (C[t,mo].B[t,mi]) (dy[t,mo].v[t,mi])
      dda_t = <G_t + Q_t, S_t>,  G_{t-1} = exp(da_t) (G_t + Q_t),  dh0 = G_0.
    v, dy [b,l,m,h,p]; da, gamma, scale [b,l,h]; B, C [b,l,m,g,n] (group form,
    dB / dC summed over the group's heads); h0, dfinal [b,h,p,n] or None.
    Returns a dict of float64 gradients (dgamma / dscale None when the weight
    is None)."""
    f = lambda t: None if t is None else np.asarray(t, np.float64)  # noqa: E731
    dy, dfinal, v, da, B, C, gamma, scale, h0 = map(f, (dy, dfinal, v, da, B, C, gamma, scale, h0))
    b, l, m, h, p = v.shape
    g, n = B.shape[3], B.shape[4]
    rep = h // g
    Bh = np.repeat(B, rep, axis=3)   # [b, l, m, h, n]
    Ch = np.repeat(C, rep, axis=3)
    gam = np.ones((b, l, h)) if gamma is None else gamma
    scl = np.ones((b, l, h)) if scale is None else scale
    S = np.zeros((l, b, h, p, n))
    hc = np.zeros((b, h, p, n)) if h0 is None else h0.copy()
    for t in range(l):
        S[t] = np.exp(da[:, t])[:, :, None, None] * hc
        hc = S[t] + scl[:, t][:, :, None, None] * np.einsum("bmhp,bmhn->bhpn", v[:, t], Bh[:, t])
    G = np.zeros((b, h, p, n)) if dfinal is None else dfinal.copy()
    dv = np.zeros_like(v)
    dBh = np.zeros_like(Bh)
    dCh = np.zeros_like(Ch)
    dda = np.zeros_like(da)
    dgam = np.zeros_like(da)
    dscl = np.zeros_like(da)
    for t in range(l - 1, -1, -1):
        vt, Bt, Ct, yt = v[:, t], Bh[:, t], Ch[:, t], dy[:, t]        # [b, m, h, .]
        Qt = np.einsum("bohp,bohn->bhpn", yt, Ct)
        yv = np.einsum("bohp,bihp->bhoi", yt, vt)                      # dy[mo] . v[mi]
        cb = np.einsum("bohn,bihn->bhoi", Ct, Bt)                      # C[mo] . B[mi]
        dCh[:, t] = np.einsum("bhpn,bohp->bohn", S[t], yt) + \
            np.einsum("bh,bhoi,bihn->bohn", gam[:, t], yv, Bt)
        GB = np.einsum("bhpn,bihn->bihp", G, Bt)                       # G_t B[t,mi]
        dBh[:, t] = np.einsum("bh,bhpn,bihp->bihn", scl[:, t], G, vt) + \
            np.einsum("bh,bhoi,bohn->bihn", gam[:, t], yv, Ct)
        dv[:, t] = scl[:, t][:, None, :, None] * GB + np.einsum("bh,bhoi,bohp->bihp", gam[:, t], cb, yt)
        dscl[:, t] = np.einsum("bihp,bihp->bh", vt, GB)
        dgam[:, t] = np.einsum("bhoi,bhoi->bh", cb, yv)
        dda[:, t] = np.einsum("bhpn,bhpn->bh", G + Qt, S[t])
        G = np.exp(da[:, t])[:, :, None, None] * (G + Qt)
    return dict(dv=dv, dda=dda, dB=dBh.reshape(b, l, m, g, rep, n).sum(4),
                dC=dCh.reshape(b, l, m, g, rep, n).sum(4), dgamma=None if gamma is None else dgam,
                dscale=None if scale is None else dscl, dh0=G)


# --------------------------------------------------------------------------
# Mamba-1 selective scan (src/mamba1/mamba1.rs:422-523, :666-733)
# --------------------------------------------------------------------------

def mamba1_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                h0=None, prec=64):
    """u,delta,z[b,d,l] A[d,n] B,C[b,n,l] D[d] h0[b,d,n] -> (y[b,d,l], hT[b,d,n])."""
    u, delta, A, B, C, D, z, delta_bias, h0 = map(_f32, (u, delta, A, B, C, D, z, delta_bias, h0))
    b, d, l = u.shape
    n = A.shape[1]
    assert delta.shape == u.shape and B.shape == C.shape == (b, n, l) and A.shape == (d, n)
    y = np.zeros_like(u)
    hT = np.zeros((b, d, n), np.float32)
    _fn("mamba1_scan", prec)(b, d, l, n, _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D),
                             _ptr(z), _ptr(delta_bias), int(bool(delta_softplus)), _ptr(h0),
                             _ptr(y), _ptr(hT))
    return y, hT


def mamba1_step(u, delta, A, B, C, state, D=None, z=None, delta_bias=None, delta_softplus=False,
                prec=64):
    """One token: u,delta,z[b,d] B,C[b,n] state[b,d,n] -> (y[b,d], new_state)."""
    u, delta, A, B, C, D, z, delta_bias = map(_f32, (u, delta, A, B, C, D, z, delta_bias))
    st = np.array(state, dtype=np.float32, copy=True)
    b, d = u.shape
    n = A.shape[1]
    y = np.zeros_like(u)
    _fn("mamba1_step", prec)(b, d, n, _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D),
                             _ptr(z), _ptr(delta_bias), int(bool(delta_softplus)), _ptr(st), _ptr(y))
    return y, st


# --------------------------------------------------------------------------
# Mamba-2 block step (src/mamba2/mamba2.rs:820-1004)
# --------------------------------------------------------------------------

def mamba2_step_ssm(zxbcdt, conv_state, conv_w, conv_b, dt_bias, A, D, norm_w, ssm_state,
                    nheads, headdim, ngroups, dstate, dt_limit=(0.0, 65504.0), norm_before_gate=False,
                    prec=64):
    """Everything of Mamba2::step between in_proj and out_proj.

    Returns (out[b, d_inner], new_conv_state, new_ssm_state)."""
    zxbcdt, conv_w, conv_b, dt_bias, A, D, norm_w = map(
        _f32, (zxbcdt, conv_w, conv_b, dt_bias, A, D, norm_w))
    cs = np.array(conv_state, dtype=np.float32, copy=True)
    ss = np.array(ssm_state, dtype=np.float32, copy=True)
    b = zxbcdt.shape[0]
    k = conv_w.shape[1]
    out = np.zeros((b, nheads * headdim), np.float32)
    _fn("mamba2_step_ssm", prec)(b, nheads, headdim, ngroups, dstate, k, _ptr(zxbcdt), _ptr(cs),
                                 _ptr(conv_w), _ptr(conv_b), _ptr(dt_bias), _ptr(A), _ptr(D),
                                 ctypes.c_float(dt_limit[0]), ctypes.c_float(dt_limit[1]),
                                 _ptr(norm_w), _ptr(ss), _ptr(out), int(bool(norm_before_gate)))
    return out, cs, ss


def conv1d_step(x, state, w, bias=None, silu=True, prec=64):
    """One depthwise causal conv step: x[b,c], state[b,c,K] -> (out[b,c], new state)."""
    x, w, bias = _f32(x), _f32(w), _f32(bias)
    st = np.array(state, dtype=np.float32, copy=True)
    b, c, k = st.shape
    out = np.zeros((b, c), np.float32)
    _fn("conv1d_step", prec)(b, c, k, _ptr(x), _ptr(st), _ptr(w), _ptr(bias), int(bool(silu)), _ptr(out))
    return out, st


def mamba1_block_step(x, p, conv_state, ssm_state, prec=64):
    """Mamba1::step (src/mamba1/mamba1.rs:533-612): in_proj -> split (xs, res) ->
    conv step + SiLU -> x_proj -> split (dt, B, C) -> dt_proj (+bias) -> softplus ->
    selective_scan_step -> * silu(res) -> out_proj.  Returns (y, conv', ssm')."""
    d_inner = p["conv_w"].shape[0]
    r = p["dt_proj_w"].shape[0]
    n = p["A"].shape[1]
    xr = linear(x, p["in_proj_w"], None, prec)
    u, cs = conv1d_step(xr[:, :d_inner], conv_state, p["conv_w"], p["conv_b"], True, prec)
    x_dbl = linear(u, p["x_proj_w"], None, prec)
    delta = linear(np.ascontiguousarray(x_dbl[:, :r]), p["dt_proj_w"], None, prec)
    y, ss = mamba1_step(u, delta, p["A"], x_dbl[:, r:r + n], x_dbl[:, r + n:], ssm_state, p["D"],
                        xr[:, d_inner:], p["dt_proj_b"], True, prec)
    return linear(y, p["out_proj_w"], None, prec), cs, ss


def mamba1_block_fwd(x, p, conv_state, ssm_state, prec=64):
    """Mamba1::forward (src/mamba1/mamba1.rs:278-352): in_proj -> split (xs, res)
    -> causal depthwise conv over [cached window[:, :, 1:] | xs] + bias, SiLU
    (:300-340; the window becomes the padded input's last K columns) -> ssm
    (:366-399: x_proj -> split (dt, B, C) -> dt_proj (+bias) -> softplus ->
    selective_scan with D u) -> * silu(res) -> out_proj.
    x [b, l, d_model] -> (y [b, l, d_model], conv' [b, d_inner, K], ssm' [b, d_inner, n])."""
    x = np.asarray(x, np.float32)
    b, L, dm = x.shape
    di = p["conv_w"].shape[0]
    r = p["dt_proj_w"].shape[0]
    n = p["A"].shape[1]
    xr = linear(x.reshape(b * L, dm), p["in_proj_w"], None, prec).reshape(b, L, 2 * di)
    # the conv of the Mamba-2 prologue with no dt heads is the same padded
    # causal conv + SiLU + window update
    u, _, cs = mamba2_conv_fwd(xr, p["conv_w"], p["conv_b"], conv_state, np.zeros(0), 0, 0, di, 0)
    u = u.astype(np.float32)
    x_dbl = linear(u.reshape(b * L, di), p["x_proj_w"], None, prec)
    delta = linear(np.ascontiguousarray(x_dbl[:, :r]), p["dt_proj_w"], None, prec).reshape(b, L, di)
    x_dbl = x_dbl.reshape(b, L, r + 2 * n)

    def bdl(t):  # [b, l, c] -> [b, c, l]
        return np.ascontiguousarray(np.asarray(t).transpose(0, 2, 1))

    y, ss = mamba1_scan(bdl(u), bdl(delta), p["A"], bdl(x_dbl[..., r:r + n]), bdl(x_dbl[..., r + n:]), p["D"],
                        bdl(xr[..., di:]), p["dt_proj_b"], True, ssm_state, prec)
    out = linear(bdl(y).reshape(b * L, di), p["out_proj_w"], None, prec)
    return out.reshape(b, L, dm), cs.astype(np.float32), ss


def rmsnorm(x, w, prec=64):
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    _fn("rmsnorm", prec)(x.shape[0], x.shape[1], _ptr(x), _ptr(w), _ptr(out))
    return out


def linear(x, W, bias=None, prec=64):
    """x[r,k] @ W[k,c] (+bias) — Burn Linear (weight stored [d_in, d_out])."""
    x, W, bias = _f32(x), _f32(W), _f32(bias)
    out = np.zeros((x.shape[0], W.shape[1]), np.float32)
    _fn("linear", prec)(x.shape[0], x.shape[1], W.shape[1], _ptr(x), _ptr(W), _ptr(bias), _ptr(out))
    return out


def mamba2_layer_step(u, params, conv_state, ssm_state, cfg, prec=64):
    """Pre-norm Layer step around Mamba2::step (src/modules/layer.rs:224-232):
    returns (u + out_proj(ssm(in_proj(RMSNorm(u)))), conv_state', ssm_state')."""
    normed = rmsnorm(u, params["pre_norm_w"], prec)
    zxbcdt = linear(normed, params["w_in"], None, prec)
    out, cs, ss = mamba2_step_ssm(zxbcdt, conv_state, params["conv_w"], params["conv_b"],
                                  params["dt_bias"], params["A"], params["D"], params["norm_w"],
                                  ssm_state, cfg["nheads"], cfg["headdim"], cfg["ngroups"],
                                  cfg["dstate"], prec=prec)
    y = linear(out, params["w_out"], None, prec)
    return u + y, cs, ss


# --------------------------------------------------------------------------
# Mamba-3 single-pass SSD (src/mamba3/single_ssd/ssd/serial.rs:56-268)
# --------------------------------------------------------------------------

def ssd3_double(v, da, B, C, h0=None, chunk=64):
    """Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated, f64 numpy,
    following its K1-K5 (src/mamba3/double_ssd/ssd/serial.rs:118-409):
    v[b,l,m,h,p] (pre-scaled) da[b,l,h] B,C[b,l,m,h,n] h0[b,h,p,n] -> (y, hT).
    The sequence is zero-padded to whole chunks (double_ssd/double_ssd/mod.rs:215-245);
    K1 cumsum of da per chunk; K2 C.B^T on the fused (step, rank) axis; K3
    chunk states with exp(cs_end - cs) v (x) B; K4 the serial state passing;
    K5 exp(cs_i) C_i h_in + (C.B^T * exp(cs_i - cs_j), kept where step(j) <=
    step(i): the triu(1) step mask of serial.rs:366-398) @ v."""
    v, da, B, C = (np.asarray(t, np.float64) for t in (v, da, B, C))
    b, l, m, h, p = v.shape
    n = B.shape[-1]
    assert B.shape == C.shape == (b, l, m, h, n) and da.shape == (b, l, h)
    Q = int(chunk)
    nch = -(-l // Q)
    L = nch * Q
    pad = L - l

    def padl(t):
        return np.concatenate([t, np.zeros((b, pad) + t.shape[2:])], 1) if pad else t

    v, da, B, C = map(padl, (v, da, B, C))
    # fused index f = step * m + rank inside a chunk
    vf = v.reshape(b, nch, Q * m, h, p).transpose(0, 1, 3, 2, 4)     # [b, c, h, QM, p]
    Bf = B.reshape(b, nch, Q * m, h, n).transpose(0, 1, 3, 2, 4)     # [b, c, h, QM, n]
    Cf = C.reshape(b, nch, Q * m, h, n).transpose(0, 1, 3, 2, 4)
    cs = np.cumsum(da.reshape(b, nch, Q, h), axis=2).transpose(0, 1, 3, 2)   # K1 [b, c, h, Q]
    end = cs[..., -1]                                                  # [b, c, h]
    csf = np.repeat(cs, m, axis=3)                                     # [b, c, h, QM]
    cb = Cf @ Bf.transpose(0, 1, 2, 4, 3)                              # K2 [b, c, h, QM, QM]
    states = (np.exp(end[..., None] - csf)[..., None] * vf).transpose(0, 1, 2, 4, 3) @ Bf  # K3 [b,c,h,p,n]
    hin = np.zeros((b, nch, h, p, n))                                  # K4
    run = np.zeros((b, h, p, n)) if h0 is None else np.asarray(h0, np.float64)
    for c in range(nch):
        hin[:, c] = run
        run = np.exp(end[:, c])[..., None, None] * run + states[:, c]
    step = np.repeat(np.arange(Q), m)
    keep = step[None, :] <= step[:, None]                              # [QM target, QM source]
    diff = csf[..., :, None] - csf[..., None, :]
    decay = np.where(keep, np.exp(np.where(keep, diff, 0.0)), 0.0)
    blue = np.exp(csf)[..., None] * (Cf @ hin.transpose(0, 1, 2, 4, 3))  # [b, c, h, QM, p]
    orange = (cb * decay) @ vf
    y = (blue + orange).transpose(0, 1, 3, 2, 4).reshape(b, L, m, h, p)[:, :l]
    return y, run


def ssd3(v, da, B, C, gamma, scale, h0=None, chunk=64, form="serial", prec=64):
    """v[b,l,m,h,p] da,gamma,scale[b,l,h] B,C[b,l,m,h,n] h0[b,h,p,n] -> (y[b,l,m,h,p], hT)."""
    v, da, B, C, gamma, scale, h0 = map(_f32, (v, da, B, C, gamma, scale, h0))
    b, l, m, h, p = v.shape
    n = B.shape[-1]
    assert B.shape == C.shape == (b, l, m, h, n) and da.shape == gamma.shape == scale.shape == (b, l, h)
    y = np.zeros_like(v)
    hT = np.zeros((b, h, p, n), np.float32)
    args = [_ptr(v), _ptr(da), _ptr(B), _ptr(C), _ptr(gamma), _ptr(scale), _ptr(h0), _ptr(y), _ptr(hT)]
    if form == "recurrent":
        _fn("ssd3_recurrent", prec)(b, l, m, h, p, n, *args)
    else:
        _fn("ssd3_serial", prec)(b, l, m, h, p, n, chunk, *args)
    return y, hT


# --------------------------------------------------------------------------
# Mamba-3 block step (src/mamba3/double_ssd/double_ssd/mod.rs:407-760)
# --------------------------------------------------------------------------

def mamba3_num_angles(rope_dim):
    """num_rope_angles (mamba3.rs:565-567): max(rope_dim / 2, 1)."""
    return max(rope_dim // 2, 1)


def mamba3_step_prep(proj, p, angle, prec=64):
    """step_project + rotate_bc_step (Complex2D) for one token.

    proj [b, 2 d_inner + 2 M G N + 3 H + A]; p: dict of heads/headdim/ngroups/dstate/
    mimo/rope_dim, dt_bias[H], a_floor, dt_limit, rotation_range, b_norm_w/c_norm_w[N],
    b_bias/c_bias[H, M, N]; angle [b, H, A] (not modified).
    Returns dict(B, C [b, M, H, N], dt, alpha, beta, gamma [b, H], angle [b, H, A])."""
    H, P, G, N, M, R = (p[k] for k in ("nheads", "headdim", "ngroups", "dstate", "mimo", "rope_dim"))
    proj = _f32(proj)
    b = proj.shape[0]
    ang = np.array(angle, dtype=np.float32, copy=True)
    Bo = np.zeros((b, M, H, N), np.float32)
    Co = np.zeros((b, M, H, N), np.float32)
    dt, al, be, ga = (np.zeros((b, H), np.float32) for _ in range(4))
    lo, hi = p.get("dt_limit", (0.0, 65504.0))
    _fn("mamba3_step_prep", prec)(b, H, P, G, N, M, R, _ptr(proj), _ptr(_f32(p["dt_bias"])),
                                  ctypes.c_float(p.get("a_floor", 1e-4)), ctypes.c_float(lo), ctypes.c_float(hi),
                                  ctypes.c_float(p.get("rotation_range", 2.0)), _ptr(_f32(p["b_norm_w"])),
                                  _ptr(_f32(p["c_norm_w"])), _ptr(_f32(p["b_bias"])), _ptr(_f32(p["c_bias"])),
                                  _ptr(ang), _ptr(Bo), _ptr(Co), _ptr(dt), _ptr(al), _ptr(be), _ptr(ga))
    return dict(B=Bo, C=Co, dt=dt, alpha=al, beta=be, gamma=ga, angle=ang)


def mamba3_step_core(x, v_state, B, K, C, alpha, beta, gamma, state, mimo_x=None, D=None, prec=64):
    """The token state update + readout: x, v_state [b, H, P]; B, K, C [b, M, H, N];
    alpha/beta/gamma [b, H]; state [b, H, P, N]; mimo_x [H, M, P] or None (M == 1).
    Returns (out [b, M, H, P] with the D skip, new state)."""
    x, v_state, B, K, C, alpha, beta, gamma, mimo_x, D = map(
        _f32, (x, v_state, B, K, C, alpha, beta, gamma, mimo_x, D))
    st = np.array(state, dtype=np.float32, copy=True)
    b, H, P, N = st.shape
    M = B.shape[1]
    out = np.zeros((b, M, H, P), np.float32)
    _fn("mamba3_step_core", prec)(b, H, P, N, M, _ptr(x), _ptr(v_state), _ptr(B), _ptr(K), _ptr(C),
                                  _ptr(alpha), _ptr(beta), _ptr(gamma), _ptr(mimo_x), _ptr(D), _ptr(st),
                                  _ptr(out))
    return out, st


def mamba3_step_finish(out, z, mimo_z=None, mimo_o=None, norm_w=None, prec=64):
    """step_finish before out_proj: out [b, M, H, P]; z [b, H*P] -> y [b, H*P]."""
    out, z, mimo_z, mimo_o, norm_w = map(_f32, (out, z, mimo_z, mimo_o, norm_w))
    b, M, H, P = out.shape
    y = np.zeros((b, H * P), np.float32)
    _fn("mamba3_step_finish", prec)(b, H, P, M, _ptr(out), _ptr(z), _ptr(mimo_z), _ptr(mimo_o),
                                    _ptr(norm_w), _ptr(y))
    return y


def mamba3_step(proj, p, cache, prec=64):
    """Mamba3::step between in_proj and out_proj (double_ssd/double_ssd/mod.rs:634-760).
    cache: dict(ssm [b,H,P,N], k_state [b,M,H,N], v_state [b,H,P], angle [b,H,A]).
    Returns (y [b, H*P], new cache); the new k_state is the rotated B, v_state the raw x."""
    H, P = p["nheads"], p["headdim"]
    proj = _f32(proj)
    b = proj.shape[0]
    d_inner = H * P
    z = proj[:, :d_inner]
    x = proj[:, d_inner:2 * d_inner].reshape(b, H, P)
    pr = mamba3_step_prep(proj, p, cache["angle"], prec)
    out, st = mamba3_step_core(x, cache["v_state"], pr["B"], cache["k_state"], pr["C"], pr["alpha"],
                               pr["beta"], pr["gamma"], cache["ssm"], p.get("mimo_x"), p.get("D"), prec)
    y = mamba3_step_finish(out, z, p.get("mimo_z"), p.get("mimo_o"), p.get("out_norm_w"), prec)
    return y, dict(ssm=st, k_state=pr["B"], v_state=np.ascontiguousarray(x), angle=pr["angle"])



# --------------------------------------------------------------------------
# Mamba-3 prefill around the single-SSD seam (single_ssd/single_ssd/mod.rs:44-360)
# --------------------------------------------------------------------------

def mamba3_prep_fwd(proj, p, cache):
    """forward_single_ssd steps 2-6 (single_ssd/single_ssd/mod.rs:86-262) in
    float64 numpy: trapezoidal_coefficients (helpers.rs:42-73), scale_t =
    gamma_t + (1 - lambda_{t+1}) dt_{t+1} (:129-150), qk_norm_expand_bias
    (helpers.rs:82-95), rotate_bc_forward Complex2D (rotation/mod.rs:653-679:
    cumulative angle = prev + cumsum_s(dt range pi tanh(rot)), wrapped only for
    cos/sin and for the cache), v = x mimo_x (helpers.rs:152-168) and the beta
    seed h0 = ssm + (dt_0 - gamma_0) sum_m (v_prev mimo_x[m]) (x) K_prev[m]
    (:195-225).  proj [b, s, row]; cache: ssm/k_state/v_state/angle.
    Returns dict(v [b,s,M,H,P], B, C [b,s,M,H,N], da, gamma, scale [b,s,H], h0, and
    the new k_state / v_state / angle)."""
    H, P, G, N, M, R = (p[k] for k in ("nheads", "headdim", "ngroups", "dstate", "mimo", "rope_dim"))
    proj = np.asarray(proj, np.float64)
    b, s, _ = proj.shape
    A = mamba3_num_angles(R)
    d_inner, bc = H * P, M * G * N
    x = proj[..., d_inner:2 * d_inner].reshape(b, s, H, P)
    braw = proj[..., 2 * d_inner:2 * d_inner + bc].reshape(b, s, M, G, N)
    craw = proj[..., 2 * d_inner + bc:2 * d_inner + 2 * bc].reshape(b, s, M, G, N)
    o = 2 * d_inner + 2 * bc
    dd_dt, dd_a, lam_raw, rot = proj[..., o:o + H], proj[..., o + H:o + 2 * H], proj[..., o + 2 * H:o + 3 * H], \
        proj[..., o + 3 * H:o + 3 * H + A]

    def softplus(v):
        return np.where(v > 18.0, v, np.log1p(np.exp(np.minimum(v, 18.0))))
    lo, hi = p.get("dt_limit", (0.0, 65504.0))
    dt = np.clip(softplus(dd_dt + np.asarray(p["dt_bias"], np.float64)), lo, hi)
    a = -np.maximum(softplus(dd_a), p.get("a_floor", 1e-4))
    da = dt * a
    lam = 1.0 / (1.0 + np.exp(-lam_raw))
    gamma = lam * dt
    nxt = np.concatenate([(1 - lam[:, 1:]) * dt[:, 1:], np.zeros((b, 1, H))], 1)
    scale = gamma + nxt

    def qk(raw, w, bias):
        rms = np.sqrt((raw * raw).mean(-1, keepdims=True) + 8.1584695e-8)
        normed = raw / rms * np.asarray(w, np.float64)                      # [b, s, M, G, N]
        exp = np.repeat(normed, H // G, axis=3)                              # group h // (H/G)
        return exp + np.asarray(bias, np.float64).transpose(1, 0, 2)[None, None]  # [b, s, M, H, N]
    Bq, Cq = qk(braw, p["b_norm_w"], p["b_bias"]), qk(craw, p["c_norm_w"], p["c_bias"])
    inc = dt[..., None] * (np.tanh(rot)[:, :, None, :] * (p.get("rotation_range", 2.0) * np.pi))  # [b,s,H,A]
    theta = np.asarray(cache["angle"], np.float64)[:, None] + np.cumsum(inc, axis=1)
    if R > 0:
        k = np.arange(R // 2)
        i0 = 2 * k if M == 1 else k
        i1 = i0 + (1 if M == 1 else N // 2)
        th = theta[:, :, None, :, :R // 2]
        cs, sn = np.cos(th), np.sin(th)
        for Z in (Bq, Cq):
            x0, x1 = Z[..., i0].copy(), Z[..., i1].copy()
            Z[..., i0] = cs * x0 - sn * x1
            Z[..., i1] = sn * x0 + cs * x1
    mx = np.ones((H, M, P)) if p.get("mimo_x") is None else np.asarray(p["mimo_x"], np.float64)
    v = x[:, :, None] * mx.transpose(1, 0, 2)[None, None]                   # [b, s, M, H, P]
    vprev = np.asarray(cache["v_state"], np.float64)[:, None] * mx.transpose(1, 0, 2)[None]  # [b, M, H, P]
    seed = np.einsum("bmhp,bmhn->bhpn", vprev, np.asarray(cache["k_state"], np.float64))
    h0 = np.asarray(cache["ssm"], np.float64) + (dt[:, 0] - gamma[:, 0])[:, :, None, None] * seed
    wrap = lambda t: t - np.round(t / (2 * np.pi)) * (2 * np.pi)  # noqa: E731
    f = lambda t: np.ascontiguousarray(t, np.float32)  # noqa: E731
    return dict(v=f(v), B=f(Bq), C=f(Cq), da=f(da), gamma=f(gamma), scale=f(scale), dt=f(dt), h0=f(h0),
                k_state=f(Bq[:, -1]), v_state=f(x[:, -1]), angle=f(wrap(theta[:, -1])))


def mamba3_finish_fwd(y_ssd, v, z, p):
    """forward_single_ssd step 9 before out_proj (single_ssd/single_ssd/mod.rs:288-332):
    y += D v, then the gate (or per-head gated norm) and the mimo_o merge per
    position.  y_ssd, v [b, s, M, H, P]; z [b, s, H*P] -> [b, s, H*P]."""
    y_ssd, v, z = (np.asarray(t, np.float32) for t in (y_ssd, v, z))
    b, s, M, H, P = y_ssd.shape
    D = np.zeros(H, np.float32) if p.get("D") is None else np.asarray(p["D"], np.float32)
    out = (y_ssd + D[None, None, None, :, None] * v).reshape(b * s, M, H, P)
    y = mamba3_step_finish(out, z.reshape(b * s, H * P), p.get("mimo_z"), p.get("mimo_o"), p.get("out_norm_w"))
    return y.reshape(b, s, H * P)


def mamba2_conv_fwd(proj, conv_w, conv_b, conv_state, dt_bias, xbc_offset, dt_offset, channels, nheads,
                    dt_limit=(0.0, 65504.0)):
    """Mamba2::forward steps 2 and 4 (src/mamba2/mamba2.rs:618-699) in float64.

    The causal depthwise conv over xpad = [conv_state[:, :, 1:] | xBC] (valid,
    :634-645, Conv1d cross-correlation) + bias, then SiLU; dt = clamp(softplus(
    dt_raw + dt_bias)) (:695, softplus threshold 18 as for f32).  The new conv
    window is the last `kernel` columns of xpad (:652-655).
    proj [b, l, row] -> (xbc [b, l, channels], dt [b, l, nheads], conv_state' [b, channels, K])."""
    proj = np.asarray(proj, np.float64)
    w = np.asarray(conv_w, np.float64)
    b, L, _ = proj.shape
    K = w.shape[1]
    x = proj[:, :, xbc_offset:xbc_offset + channels]
    tail = np.asarray(conv_state, np.float64)[:, :, 1:].transpose(0, 2, 1)
    pad = np.concatenate([tail, x], axis=1)  # [b, K - 1 + L, channels]
    acc = np.zeros((b, L, channels))
    if conv_b is not None:
        acc += np.asarray(conv_b, np.float64)
    for k in range(K):
        acc += pad[:, k:k + L, :] * w[:, k]
    xbc = acc / (1.0 + np.exp(-acc))
    new_state = np.ascontiguousarray(pad[:, L - 1:L - 1 + K, :].transpose(0, 2, 1))
    raw = proj[:, :, dt_offset:dt_offset + nheads] + np.asarray(dt_bias, np.float64)
    sp = np.where(raw > 18.0, raw, np.log1p(np.exp(np.minimum(raw, 18.0))))
    dt = np.clip(sp, dt_limit[0], dt_limit[1])
    return xbc, dt, new_state


def mamba2_gated_rmsnorm(y, z, gamma, eps, norm_before_gate=False):
    """RmsNormGated::forward (src/modules/norm/rms_norm_gated.rs:70-135) over the
    last axis in float64: gate-then-norm (default) or norm-then-gate."""
    y = np.asarray(y, np.float64)
    z = np.asarray(z, np.float64)
    sz = z / (1.0 + np.exp(-z))
    g = y if norm_before_gate else y * sz
    out = g / np.sqrt(np.mean(g * g, axis=-1, keepdims=True) + eps) * np.asarray(gamma, np.float64)
    return out * sz if norm_before_gate else out


def mamba2_block_fwd(proj, p, conv_state, ssm_state, chunk, cfg, eps=8.1584695e-8, io_round=None):
    """Mamba2::forward between in_proj and out_proj (src/mamba2/mamba2.rs:546-786):
    conv prologue -> SSD (ssd2, f64) -> gated RMSNorm with z.  proj [b, l, row];
    p has conv_w, conv_b, dt_bias, A, D, norm_w.  Returns (y [b, l, d_inner],
    conv_state', ssm_state').  ``io_round`` (e.g. a bf16 rounding) is applied
    where a model of that dtype stores a tensor: the conv output, the SSD's y
    and the normed output."""
    rnd = io_round if io_round is not None else (lambda a: a)
    H, P, G, N = cfg["nheads"], cfg["headdim"], cfg["ngroups"], cfg["dstate"]
    d_inner = H * P
    conv_dim = d_inner + 2 * G * N
    b, L, _ = proj.shape
    xbc, dt, cs = mamba2_conv_fwd(proj, p["conv_w"], p.get("conv_b"), conv_state, p["dt_bias"], d_inner,
                                  d_inner + conv_dim, conv_dim, H, cfg.get("dt_limit", (0.0, 65504.0)))
    xbc = rnd(xbc)
    x = xbc[:, :, :d_inner].reshape(b, L, H, P)
    Bm = xbc[:, :, d_inner:d_inner + G * N].reshape(b, L, G, N)
    Cm = xbc[:, :, d_inner + G * N:].reshape(b, L, G, N)
    y, hT = ssd2(x, dt, p["A"], Bm, Cm, p.get("D"), ssm_state, chunk=chunk)
    y = rnd(y)
    z = np.asarray(proj, np.float64)[:, :, :d_inner]
    yn = mamba2_gated_rmsnorm(np.asarray(y, np.float64).reshape(b, L, d_inner), z, p["norm_w"], eps,
                              cfg.get("norm_before_gate", False))
    return rnd(yn), cs, hT
