"""Seeded synthetic inputs with the distributions of BASELINE.json's configs.

Shared by the tests, the golden-fixture script, smoke() and bench.py.  All
generators use numpy.random.default_rng(seed) so every run is reproducible.
"""

from __future__ import annotations

import numpy as np


def softplus(v):
    return np.where(v > 18.0, v, np.log1p(np.exp(np.minimum(v, 18.0))))


def inv_softplus(y):
    return y + np.log(-np.expm1(-y))


def ssd2_inputs(seed, b, l, h, p, g, n, h0=False, d=True, dt_range=(1e-3, 0.1)):
    """Config-0 distributions:
    x~N(0,1); dt = softplus(N(0,1) + b_h), b_h = softplus^-1(exp(U(ln lo, ln hi)))
    (the reference's dt_bias init, mamba2.rs:443-453); A = -exp(U(ln1, ln16));
    B,C ~ N(0,1)/sqrt(n); D~N(0,1); h0 ~ N(0, 0.1) when requested."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, l, h, p), dtype=np.float32)
    bias = inv_softplus(np.exp(rng.uniform(np.log(dt_range[0]), np.log(dt_range[1]), h)))
    dt = softplus(rng.standard_normal((b, l, h)) + bias[None, None, :]).astype(np.float32)
    A = (-np.exp(rng.uniform(0.0, np.log(16.0), h))).astype(np.float32)
    B = (rng.standard_normal((b, l, g, n)) / np.sqrt(n)).astype(np.float32)
    C = (rng.standard_normal((b, l, g, n)) / np.sqrt(n)).astype(np.float32)
    D = rng.standard_normal(h).astype(np.float32) if d else None
    hs = (0.1 * rng.standard_normal((b, h, p, n))).astype(np.float32) if h0 else None
    return dict(x=x, dt=dt, A=A, B=B, C=C, D=D, h0=hs)


def ssd2_test_inputs(seed, b, l, h, p, g, n, h0=True):
    """The reference's own test distributions (src/mamba2/ssd/ssd_path/tests.rs:33-67):
    x~N(0,1); dt~U(0.05,0.3); A~U(-1,-0.5); B,C~N(0,1); D~N(0,0.1); h0~N(0,0.1)."""
    rng = np.random.default_rng(seed)
    return dict(
        x=rng.standard_normal((b, l, h, p), dtype=np.float32),
        dt=rng.uniform(0.05, 0.3, (b, l, h)).astype(np.float32),
        A=rng.uniform(-1.0, -0.5, h).astype(np.float32),
        B=rng.standard_normal((b, l, g, n), dtype=np.float32),
        C=rng.standard_normal((b, l, g, n), dtype=np.float32),
        D=(0.1 * rng.standard_normal(h)).astype(np.float32),
        h0=(0.1 * rng.standard_normal((b, h, p, n))).astype(np.float32) if h0 else None,
    )


def bf16_round(a):
    """Round-to-nearest-even to bf16, returned as float32 (exact bf16 values)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def mamba1_inputs(seed, b, d, l, n, h0=False):
    """Config-2 distributions: u~N(0,1) [b,d,l]; delta = softplus(N(0,1)-4);
    A = -(1..n) per channel (S4D-real, mamba1.rs:184-194); B,C~N(0,1) [b,n,l];
    D = 1; z~N(0,1)."""
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((b, d, l), dtype=np.float32)
    delta = softplus(rng.standard_normal((b, d, l)) - 4.0).astype(np.float32)
    A = np.tile(-np.arange(1, n + 1, dtype=np.float32), (d, 1))
    B = rng.standard_normal((b, n, l), dtype=np.float32)
    C = rng.standard_normal((b, n, l), dtype=np.float32)
    D = np.ones(d, np.float32)
    z = rng.standard_normal((b, d, l), dtype=np.float32)
    hs = (0.1 * rng.standard_normal((b, d, n))).astype(np.float32) if h0 else None
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, h0=hs)


def ssd3_inputs(seed, b, l, m, h, p, n, lam=None):
    """Mamba-3 single-SSD inputs: v, per-head B/C, da = dt A, gamma = lam dt,
    scale = gamma_t + (1 - lam_{t+1}) dt_{t+1} (0 past the end,
    single_ssd/single_ssd/mod.rs:129-150), beta = (1 - lam) dt exp(da), h0."""
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((b, l, m, h, p)).astype(np.float32)
    B = (rng.standard_normal((b, l, m, h, n)) / np.sqrt(n)).astype(np.float32)
    C = (rng.standard_normal((b, l, m, h, n)) / np.sqrt(n)).astype(np.float32)
    dt = rng.uniform(0.01, 0.3, (b, l, h))
    A = -rng.uniform(0.5, 2.0, h)
    lam = 1.0 / (1.0 + np.exp(-rng.standard_normal((b, l, h)))) if lam is None else np.full((b, l, h), lam)
    da = dt * A
    gamma = lam * dt
    nxt = np.concatenate([(1 - lam[:, 1:]) * dt[:, 1:], np.zeros((b, 1, h))], 1)
    scale = gamma + nxt
    beta = (1 - lam) * dt * np.exp(da)
    h0 = (0.1 * rng.standard_normal((b, h, p, n))).astype(np.float32)
    f = lambda a: np.asarray(a, np.float32)
    return dict(v=v, B=B, C=C, da=f(da), gamma=f(gamma), scale=f(scale), beta=beta, dt=dt, A=A, lam=lam, h0=h0)
