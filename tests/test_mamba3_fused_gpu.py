"""The Mamba-3 prologue fused into the single-SSD scan (mamba3_ssd_fused_fwd,
C ABI), checked on identical inputs stage by stage (single_ssd/single_ssd/mod.rs:86-290):

* the fused kernel with D = NULL equals the segment prep (mamba3_prep_fwd)
  followed by the seam scan (mamba_ssd3_fwd) bit for bit, outputs, final
  state and cache tail: both prologues form coefficients, fixed-point angles
  and B / C rows with the same arithmetic, and both scans share their core;
* the fused output (with D) matches oracle.ssd3 + D v on the prep's own bf16
  v / B / C and f32 coefficients at north_star's absolute bars (rtol 2e-2,
  atol 1e-2 on every element; y rounded to bf16 once, as the kernel stores it);
* the prep matches oracle.mamba3_prep_fwd: v exactly, B and C within one bf16
  unit (an f32 prologue carries dt and tanh in f32 through the angle
  recurrence, as the reference's f32 model does, and rounds a small fraction
  of elements to the neighbouring bf16 value of the f64 oracle's), the
  coefficients and the cache tail at f32 tolerances.

Cases: the config-4 head shape (headdim 64, dstate 128, MIMO 4, every pair
rotated) over several chunks with a ragged tail, MIMO 2 with two groups and
half the pairs rotated, MIMO 8 with the rotation off, SISO (MIMO 1: 128-step
chunks, adjacent rotation pairs) with every pair rotated and with two groups
and half the pairs rotated; split calls; the block forward taking the fused
path (MIMO 4 and SISO), and against the oracle pipeline with block-init
weights."""

import numpy as np
import pytest

from inputs import bf16_round
from test_mamba3_prefill_gpu import _cache, _cfg, _g, _gpu_cache, _params

pytestmark = pytest.mark.gpu

CASES = [
    # (b, L, H, G, M, rope_dim)
    (2, 100, 4, 1, 4, 128),   # config-4 head shape: 4 chunks of 32 steps, ragged tail
    (1, 257, 2, 1, 4, 128),   # one step past a chunk boundary
    (1, 70, 4, 2, 2, 64),     # MIMO 2 (64-step chunks), two groups, half the pairs rotated
    (2, 45, 2, 1, 8, 0),      # MIMO 8 (16-step chunks), rotation off
    (2, 300, 4, 1, 1, 128),   # SISO: 128-step chunks, ragged third chunk, every pair rotated
    (1, 129, 2, 2, 1, 64),    # SISO: one step past a chunk, two groups, half the pairs rotated
]
# the cases of the bit-for-bit comparison with the unfused sequence
EQUAL_CASES = CASES[:3] + CASES[4:]

# north_star's bar for bf16 in / f32 accumulate, element by element
BF16_TOL = dict(rtol=2e-2, atol=1e-2)


def _inputs(case):
    import torch
    b, L, H, G, M, R = case
    prm = _params(sum(case), H, 64, G, 128, M, R)
    cfg = _cfg(prm)
    rng = np.random.default_rng(sum(case) + 1)
    proj = torch.from_numpy(rng.standard_normal((b, L, cfg.d_in_proj)).astype(np.float32)).to(torch.bfloat16)
    cache = _cache(sum(case) + 2, b, prm, cfg.num_rope_angles)
    return prm, cfg, proj, cache


def _rows8(proj):
    """proj on the GPU with its rows padded to 8 elements (16-byte aligned row
    starts, the fused kernel's layout), as a strided view."""
    import torch
    b, L, d = proj.shape
    wide = torch.zeros((b, L, -(-d // 8) * 8), dtype=proj.dtype, device="cuda")
    wide[:, :, :d] = proj.cuda()
    return wide[:, :, :d]


def _prep_kw(prm):
    return dict(dt_bias=_g(prm, "dt_bias"), b_norm_w=_g(prm, "b_norm_w"), c_norm_w=_g(prm, "c_norm_w"),
                b_bias=_g(prm, "b_bias"), c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"))


def _run_fused(prm, cfg, proj, cache, with_d=True):
    import torch
    import mamba_hip
    cg = _gpu_cache(cache)
    a = mamba_hip.mamba3_fused_args(cfg, _rows8(proj), cg, **_prep_kw(prm), D=_g(prm, "D") if with_d else None)
    assert mamba_hip.mamba3_fused_supported(a) == 1
    y, hT = mamba_hip.mamba3_fused_run(a, cg)
    torch.cuda.synchronize()
    return y, hT, cg


def _run_prep_seam(prm, cfg, proj, cache):
    """The unfused sequence on the GPU: mamba3_prep_fwd -> mamba_ssd3_fwd."""
    import torch
    import mamba_hip
    cu = _gpu_cache(cache)
    pr = mamba_hip.mamba3_prep_fwd(cfg, _rows8(proj), cu, **_prep_kw(prm))
    ys, hs = mamba_hip.ssd3_fwd(pr["v"], pr["da"], pr["B"], pr["C"], pr["gamma"], pr["scale"], pr["h0"])
    torch.cuda.synchronize()
    return pr, ys, hs, cu


def _close(got, want, **tol):
    np.testing.assert_allclose(got, want, **(tol or BF16_TOL))


def _ulp_bf16(a):
    """One bf16 unit at each element's magnitude."""
    return np.exp2(np.floor(np.log2(np.maximum(np.abs(a), 1e-30))) - 7)


def oracle_on_prep(pr, prm, D=True, sl=slice(None)):
    """oracle.ssd3 (+ D v) on the GPU prep's own bf16 v / B / C and f32
    coefficients (batch rows `sl`), y rounded to bf16 once as the fused kernel
    stores it.  Returns (y, final state)."""
    import oracle
    f = {k: pr[k][sl].float().cpu().numpy() for k in ("v", "B", "C", "da", "gamma", "scale", "h0")}
    yo, ho = oracle.ssd3(f["v"], f["da"], f["B"], f["C"], f["gamma"], f["scale"], f["h0"], chunk=32)
    if D and prm.get("D") is not None:
        yo = yo + prm["D"][None, None, None, :, None] * f["v"]
    return bf16_round(yo), ho


# bound on the f32 angle recurrence's drift from the f64 oracle over the test
# sequences (<= 8192 steps; 2e-5 rad measured after 2048 steps)
ANGLE_DRIFT = 5e-5


def _pair_len(a, M):
    """Length of each element's rotation pair ((k, k + N/2) for MIMO > 1,
    (2k, 2k + 1) otherwise), at every element."""
    n = a.shape[-1]
    if M > 1:
        ln = np.hypot(a[..., :n // 2], a[..., n // 2:])
        return np.concatenate([ln, ln], -1)
    ln = np.hypot(a[..., 0::2], a[..., 1::2])
    return np.repeat(ln, 2, -1)


def check_prep_against_oracle(pr, cu, proj, prm, cache, sl=slice(None), flip_frac=1e-2, angle_atol=1e-4):
    """The GPU prep against oracle.mamba3_prep_fwd (f64) on batch rows `sl`:
    v exact; B and C within one bf16 unit of the oracle's rounding plus the
    angle drift's absolute reach (ANGLE_DRIFT times the element's rotation-pair
    length), with at most `flip_frac` of the elements away from the oracle's
    value; coefficients, initial state and cache tail at f32 tolerances.
    Returns the fractions of B / C elements that differ."""
    import oracle
    one = {k: v[sl] for k, v in cache.items()}
    r = oracle.mamba3_prep_fwd(proj[sl].float().numpy(), prm, one)
    np.testing.assert_array_equal(pr["v"][sl].float().cpu().numpy(), bf16_round(r["v"]))
    fracs = {}
    for k in ("B", "C"):
        got, want = pr[k][sl].float().cpu().numpy(), bf16_round(r[k])
        diff = np.abs(got - want)
        drift = ANGLE_DRIFT * _pair_len(r[k].astype(np.float64), prm["mimo"]) if prm["rope_dim"] else 0.0
        bound = _ulp_bf16(np.maximum(np.abs(got), np.abs(want))) * 1.001 + drift + 1e-6
        assert np.all(diff <= bound), (k, float(np.max(diff / bound)))
        fracs[k] = float(np.mean(diff > 0))
        assert fracs[k] <= flip_frac, (k, fracs[k])
    for k in ("da", "gamma", "scale"):
        np.testing.assert_allclose(pr[k][sl].cpu().numpy(), r[k], rtol=1e-5, atol=1e-7, err_msg=k)
    np.testing.assert_allclose(pr["h0"][sl].cpu().numpy(), r["h0"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(cu.k_state_bmhr[sl].cpu().numpy(), r["k_state"], rtol=1e-3, atol=1e-3)
    np.testing.assert_array_equal(cu.v_state_bhp[sl].cpu().numpy(), r["v_state"])
    ag = cu.angle_bha[sl].cpu().numpy()
    np.testing.assert_allclose(np.cos(ag), np.cos(r["angle"]), atol=angle_atol)
    np.testing.assert_allclose(np.sin(ag), np.sin(r["angle"]), atol=angle_atol)
    return fracs


@pytest.mark.parametrize("case", CASES)
def test_mamba3_fused_matches_oracle(case):
    print("fused vs oracle", case, flush=True)
    prm, cfg, proj, cache = _inputs(case)
    y, hT, cg = _run_fused(prm, cfg, proj, cache)
    pr, ys, hs, cu = _run_prep_seam(prm, cfg, proj, cache)
    want, ho = oracle_on_prep(pr, prm)
    _close(y.float().cpu().numpy(), want)
    _close(hT.cpu().numpy(), ho)
    fr = check_prep_against_oracle(pr, cu, proj, prm, cache)
    print("  B / C one unit from the oracle's rounding:", fr, flush=True)
    # the cache tail of the fused call is the prep's
    for nm in ("k_state_bmhr", "v_state_bhp", "angle_bha"):
        assert bool((getattr(cg, nm) == getattr(cu, nm)).all()), nm


@pytest.mark.parametrize("case", EQUAL_CASES)
def test_mamba3_fused_equals_prep_then_seam(case):
    """With D = NULL the fused kernel is the unfused sequence mamba3_prep_fwd ->
    mamba_ssd3_fwd (per-head v, B, C and coefficients in HBM), bit for bit."""
    import torch
    print("fused == prep + seam", case, flush=True)
    prm, cfg, proj, cache = _inputs(case)
    y, hT, cg = _run_fused(prm, cfg, proj, cache, with_d=False)
    pr, ys, hs, cu = _run_prep_seam(prm, cfg, proj, cache)
    assert torch.equal(y, ys), f"{int((y != ys).sum())} elements differ"
    assert torch.equal(hT, hs)
    for nm in ("k_state_bmhr", "v_state_bhp", "angle_bha"):
        assert torch.equal(getattr(cg, nm), getattr(cu, nm)), nm


def test_mamba3_fused_split_carries_cache():
    """Two fused calls (prompt, then continuation) equal one call over the
    concatenation: the final state, k_state / v_state and angle carry the
    sequence across calls through the beta seed (the fixed-point angle makes
    the B / C rows of both runs the same values; only the scan's chunking
    differs)."""
    import torch
    print("fused split", flush=True)
    case = (1, 160, 2, 1, 4, 128)
    prm, cfg, proj, cache = _inputs(case)
    y, hT, cg = _run_fused(prm, cfg, proj, cache)
    y1, h1, c1 = _run_fused(prm, cfg, proj[:, :97], cache)
    c1d = dict(ssm=h1.cpu().numpy(), k_state=c1.k_state_bmhr.cpu().numpy(), v_state=c1.v_state_bhp.cpu().numpy(),
               angle=c1.angle_bha.cpu().numpy())
    y2, h2, c2 = _run_fused(prm, cfg, proj[:, 97:], c1d)
    torch.cuda.synchronize()
    _close(torch.cat([y1, y2], 1).float().cpu().numpy(), y.float().cpu().numpy())
    _close(h2.cpu().numpy(), hT.cpu().numpy())
    np.testing.assert_array_equal(c2.v_state_bhp.cpu().numpy(), cg.v_state_bhp.cpu().numpy())


@pytest.mark.parametrize("mimo", [4, 1])
def test_mamba3_block_forward_takes_fused_path(mimo):
    """Mamba3.forward (single-ssd cache) at the config-4 head shape (and its
    SISO twin) runs the fused scan, and equals the same block through the
    unfused sequence."""
    import torch
    import mamba_hip
    from mamba_hip import mamba3 as m3mod
    print("block forward fused, mimo", mimo, flush=True)
    cfg = mamba_hip.Mamba3Config(d_model=128, state_rank=128, per_head_dim=64, mimo_rank=mimo)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    m = cfg.init("cuda", torch.bfloat16, gen)
    m.b_bias.normal_(0, 0.1, generator=gen)
    m.D.normal_(0, 1, generator=gen)
    x = torch.randn((2, 90, 128), generator=gen, device="cuda").to(torch.bfloat16)
    calls = []
    orig = m3mod.fused_run

    def spy(a, cache, events=None):
        calls.append(1)
        return orig(a, cache, events)
    m3mod.fused_run = spy
    try:
        out_f, cf = m.forward(x, None)
    finally:
        m3mod.fused_run = orig
    assert calls == [1]
    # the unfused sequence on the same block: prep -> mamba_ssd3_fwd -> finish
    proj = m._in_proj(x)
    cu = m.new_cache(2)
    pr = m3mod.prep_fwd(cfg, proj, cu, dt_bias=m.dt_bias, b_norm_w=m.b_norm_w, c_norm_w=m.c_norm_w,
                        b_bias=m.b_bias, c_bias=m.c_bias, mimo_x=m.mimo_x)
    yu, hu = mamba_hip.ssd3_fwd(pr["v"], pr["da"], pr["B"], pr["C"], pr["gamma"], pr["scale"], pr["h0"])
    yb = m3mod.finish_fwd(cfg, yu, pr["v"], proj[:, :, :cfg.d_inner], D=m.D, mimo_z=m.mimo_z, mimo_o=m.mimo_o)
    out_u = m._out_proj(yb, x)
    torch.cuda.synchronize()
    _close(out_f.float().cpu().numpy(), out_u.float().cpu().numpy())
    _close(cf.ssm_bhpr.cpu().numpy(), hu.cpu().numpy())


def _block_params(m):
    """The oracle's parameter dict of a Mamba3 block."""
    c = m.cfg
    f = lambda t: None if t is None else t.float().cpu().numpy()  # noqa: E731
    M = c.mimo_rank
    return dict(nheads=c.nheads, headdim=c.per_head_dim, ngroups=c.ngroups, dstate=c.state_rank, mimo=M,
                rope_dim=c.rope_dim, dt_bias=f(m.dt_bias), a_floor=c.a_floor, dt_limit=c.dt_limit,
                rotation_range=c.rotation_range, b_norm_w=f(m.b_norm_w), c_norm_w=f(m.c_norm_w),
                b_bias=f(m.b_bias), c_bias=f(m.c_bias), D=f(m.D), mimo_x=None if M == 1 else f(m.mimo_x),
                mimo_z=None if M == 1 else f(m.mimo_z), mimo_o=None if M == 1 else f(m.mimo_o),
                out_norm_w=f(getattr(m, "out_norm_w", None)))


def test_mamba3_block_forward_bf16_matches_oracle():
    """Mamba3.forward in bf16 at the config-4 head shape (headdim 64, dstate
    128, MIMO 4, every pair rotated), block-init weights, from an empty cache,
    against the oracle pipeline stage by stage on identical inputs: the block's
    in_proj rows against the f64 product (within one bf16 unit: the library
    GEMM's accumulation order); on those rows, the prep against
    oracle.mamba3_prep_fwd (check_prep_against_oracle); on the prep's values,
    the block's scan output y and final state against oracle.ssd3 + D v; on
    that y, the block's output against oracle.mamba3_finish_fwd -> out_proj
    (f64), rounded where the bf16 model stores a tensor.  North_star's
    absolute bars at every stage."""
    import torch
    import mamba_hip
    import oracle
    from mamba_hip import mamba3 as m3mod
    print("block forward bf16 vs oracle", flush=True)
    cfg = mamba_hip.Mamba3Config(d_model=128, state_rank=128, per_head_dim=64, mimo_rank=4)
    m = cfg.init("cuda", torch.bfloat16, torch.Generator(device="cuda").manual_seed(13))
    b, L = 2, 150
    x = torch.randn((b, L, cfg.d_model), generator=torch.Generator(device="cuda").manual_seed(14),
                    device="cuda").to(torch.bfloat16)
    out, cache = m.forward(x, None, chunk_len=32)
    prm = _block_params(m)
    f64 = lambda t: t.float().cpu().numpy().astype(np.float64)  # noqa: E731
    proj = m._in_proj(x)
    want_proj = bf16_round(f64(x) @ f64(m.in_proj_w))
    pf = proj.float().cpu().numpy()
    # one bf16 unit, or the f32 accumulation's reach (sum |x w|) near zero
    reach = 1e-6 * (np.abs(f64(x)) @ np.abs(f64(m.in_proj_w)))
    assert np.all(np.abs(pf - want_proj) <= _ulp_bf16(np.maximum(np.abs(pf), np.abs(want_proj))) * 1.001 + reach)
    c0 = _cache(0, b, prm, cfg.num_rope_angles, zero=True)
    cu = m.new_cache(b)
    pr = m3mod.prep_fwd(cfg, proj, cu, dt_bias=m.dt_bias, b_norm_w=m.b_norm_w, c_norm_w=m.c_norm_w,
                        b_bias=m.b_bias, c_bias=m.c_bias, mimo_x=m.mimo_x)
    torch.cuda.synchronize()
    check_prep_against_oracle(pr, cu, proj.cpu(), prm, c0)
    # the scan the block ran (the fused kernel on the same rows) against the oracle on the prep's values
    cf = m.new_cache(b)
    yg, _ = m3mod.fused_run(m3mod.fused_args(cfg, proj, cf, dt_bias=m.dt_bias, b_norm_w=m.b_norm_w,
                                             c_norm_w=m.c_norm_w, b_bias=m.b_bias, c_bias=m.c_bias,
                                             mimo_x=m.mimo_x, D=m.D), cf)
    torch.cuda.synchronize()
    y, ho = oracle_on_prep(pr, prm)
    yg = yg.float().cpu().numpy()
    _close(yg, y)
    _close(cache.ssm_bhpr.cpu().numpy(), ho)
    # the epilogue on that y: the gate and MIMO merge (D v is already in y), out_proj in f64
    fin = bf16_round(oracle.mamba3_finish_fwd(yg, pr["v"].float().cpu().numpy(), pf[:, :, :cfg.d_inner],
                                              dict(prm, D=None)))
    want = bf16_round(fin.astype(np.float64) @ f64(m.out_proj_w))
    _close(out.float().cpu().numpy(), want)
