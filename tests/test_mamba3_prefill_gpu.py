"""Mamba-3 prefill around the single-SSD seam: mamba3_prep_fwd and
mamba3_finish_fwd (C ABI) vs the CPU oracle (oracle.mamba3_prep_fwd, pinned
against the per-token prep and by prefill-then-steps == steps), and the
Mamba3.forward composition (prep -> mamba_ssd3_fwd -> finish) followed by
steps.  f32 at rtol 1e-4 (1e-3 through the chunked SSD); bf16 I/O at
rtol 2e-2 / atol 1e-2."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=2e-5)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _params(seed, H, P, G, N, M, rope_dim, out_norm=False):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return dict(nheads=H, headdim=P, ngroups=G, dstate=N, mimo=M, rope_dim=rope_dim,
                dt_bias=rng.uniform(-3, -1, H).astype(np.float32), a_floor=1e-4, dt_limit=(0.0, 65504.0),
                rotation_range=2.0, b_norm_w=rng.uniform(0.5, 1.5, N).astype(np.float32),
                c_norm_w=rng.uniform(0.5, 1.5, N).astype(np.float32), b_bias=0.1 * f(H, M, N),
                c_bias=0.1 * f(H, M, N), D=f(H), mimo_x=f(H, M, P) if M > 1 else None,
                mimo_z=f(H, M, P) if M > 1 else None, mimo_o=f(H, M, P) if M > 1 else None,
                out_norm_w=rng.uniform(0.5, 1.5, P).astype(np.float32) if out_norm else None)


def _cfg(prm):
    import mamba_hip
    N = prm["dstate"]
    return mamba_hip.Mamba3Config(d_model=prm["nheads"] * prm["headdim"] // 2, state_rank=N,
                                  per_head_dim=prm["headdim"], ngroups=prm["ngroups"], mimo_rank=prm["mimo"],
                                  rope_fraction=prm["rope_dim"] / N, has_outproj_norm=prm["out_norm_w"] is not None)


def _cache(seed, b, prm, A, zero=False):
    rng = np.random.default_rng(seed)
    H, P, N, M = prm["nheads"], prm["headdim"], prm["dstate"], prm["mimo"]
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    if zero:
        return dict(ssm=z(b, H, P, N), k_state=z(b, M, H, N), v_state=z(b, H, P), angle=z(b, H, A))
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return dict(ssm=0.1 * f(b, H, P, N), k_state=(f(b, M, H, N) / np.sqrt(N)).astype(np.float32),
                v_state=f(b, H, P), angle=rng.uniform(-3, 3, (b, H, A)).astype(np.float32))


def _gpu_cache(c):
    import mamba_hip
    return mamba_hip.Mamba3Cache(_t(c["ssm"]), _t(c["k_state"]), _t(c["v_state"]), _t(c["angle"]))


def _g(prm, k):
    return None if prm.get(k) is None else _t(prm[k])


CASES = [
    # (b, L, H, P, G, N, M, rope_dim)
    (2, 37, 4, 16, 2, 16, 1, 16),    # SISO, every pair rotated
    (2, 21, 4, 16, 1, 32, 4, 32),    # MIMO 4, half-and-half
    (1, 50, 2, 8, 1, 16, 2, 8),      # partial rotation, ragged tiles
    (2, 9, 4, 32, 2, 64, 1, 0),      # rotation off
]


@pytest.mark.parametrize("case", CASES)
def test_mamba3_prep_fwd_matches_oracle(case):
    import torch
    import mamba_hip
    import oracle
    b, L, H, P, G, N, M, R = case
    prm = _params(sum(case), H, P, G, N, M, R)
    cfg = _cfg(prm)
    A = cfg.num_rope_angles
    rng = np.random.default_rng(sum(case) + 1)
    proj = rng.standard_normal((b, L, cfg.d_in_proj)).astype(np.float32)
    cache = _cache(sum(case) + 2, b, prm, A)
    cg = _gpu_cache(cache)
    out = mamba_hip.mamba3_prep_fwd(cfg, _t(proj), cg, dt_bias=_g(prm, "dt_bias"), b_norm_w=_g(prm, "b_norm_w"),
                                    c_norm_w=_g(prm, "c_norm_w"), b_bias=_g(prm, "b_bias"),
                                    c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"))
    torch.cuda.synchronize()
    r = oracle.mamba3_prep_fwd(proj, prm, cache)
    for k in ("v", "B", "C", "da", "gamma", "scale", "h0"):
        np.testing.assert_allclose(out[k].cpu().numpy(), r[k], **F32_TOL, err_msg=k)
    np.testing.assert_allclose(cg.k_state_bmhr.cpu().numpy(), r["k_state"], **F32_TOL)
    np.testing.assert_allclose(cg.v_state_bhp.cpu().numpy(), r["v_state"], **F32_TOL)
    ag = cg.angle_bha.cpu().numpy()
    np.testing.assert_allclose(np.cos(ag), np.cos(r["angle"]), atol=5e-5)
    np.testing.assert_allclose(np.sin(ag), np.sin(r["angle"]), atol=5e-5)


@pytest.mark.parametrize("M,out_norm", [(1, False), (4, True), (2, False)])
def test_mamba3_finish_fwd_matches_oracle(M, out_norm):
    import torch
    import mamba_hip
    import oracle
    b, L, H, P = 2, 11, 3, 48
    prm = _params(61 + M, H, P, 1, 16, M, 16, out_norm)
    rng = np.random.default_rng(67)
    y = rng.standard_normal((b, L, M, H, P)).astype(np.float32)
    v = rng.standard_normal((b, L, M, H, P)).astype(np.float32)
    zw = rng.standard_normal((b, L, 2 * H * P)).astype(np.float32)  # z as a slice of a wider row
    z = _t(zw)[:, :, :H * P]
    out = mamba_hip.mamba3_finish_fwd(_cfg(prm), _t(y), _t(v), z, D=_g(prm, "D"), mimo_z=_g(prm, "mimo_z"),
                                      mimo_o=_g(prm, "mimo_o"), out_norm_w=_g(prm, "out_norm_w"))
    torch.cuda.synchronize()
    want = oracle.mamba3_finish_fwd(y, v, zw[:, :, :H * P], prm)
    np.testing.assert_allclose(out.cpu().numpy(), want, **F32_TOL)


def test_mamba3_prep_fwd_bf16_config4_heads():
    """bf16 in_proj rows and bf16 v/B/C outputs at the config-4 head shape."""
    import torch
    import mamba_hip
    import oracle
    b, L, H, P, G, N, M = 1, 40, 4, 64, 1, 128, 4
    prm = _params(71, H, P, G, N, M, 128)
    cfg = _cfg(prm)
    rng = np.random.default_rng(73)
    proj = torch.from_numpy(rng.standard_normal((b, L, cfg.d_in_proj)).astype(np.float32)).to(torch.bfloat16)
    cache = _cache(79, b, prm, cfg.num_rope_angles)
    out = mamba_hip.mamba3_prep_fwd(cfg, proj.cuda(), _gpu_cache(cache), dt_bias=_g(prm, "dt_bias"),
                                    b_norm_w=_g(prm, "b_norm_w"), c_norm_w=_g(prm, "c_norm_w"),
                                    b_bias=_g(prm, "b_bias"), c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"))
    torch.cuda.synchronize()
    r = oracle.mamba3_prep_fwd(proj.float().numpy(), prm, cache)
    for k in ("v", "B", "C"):
        np.testing.assert_allclose(out[k].float().cpu().numpy(), r[k], rtol=2e-2, atol=1e-2, err_msg=k)
    for k in ("da", "gamma", "scale", "h0"):
        np.testing.assert_allclose(out[k].cpu().numpy(), r[k], **F32_TOL, err_msg=k)


@pytest.mark.parametrize("M", [1, 4])
def test_mamba3_forward_then_step(M):
    """Mamba3.forward over a prompt (in_proj -> prep -> mamba_ssd3_fwd ->
    finish -> out_proj) and then Mamba3.step on its cache, against the oracle
    pipeline with the same products."""
    import torch
    import mamba_hip
    import oracle
    cfg = mamba_hip.Mamba3Config(d_model=64, state_rank=32, per_head_dim=16, mimo_rank=M, rope_fraction=0.5)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5 + M)
    m = cfg.init("cuda", torch.float32, gen)
    m.b_bias.normal_(0, 0.1, generator=gen)
    m.D.normal_(0, 1, generator=gen)
    b, L = 2, 23
    x = torch.randn((b, L, 64), generator=gen, device="cuda")
    xt = torch.randn((b, 64), generator=gen, device="cuda")
    out, cache = m.forward(x, None, chunk_len=8)
    out2, cache = m.step(xt, cache)
    torch.cuda.synchronize()
    prm = dict(nheads=cfg.nheads, headdim=16, ngroups=1, dstate=32, mimo=M, rope_dim=cfg.rope_dim,
               dt_bias=m.dt_bias.cpu().numpy(), a_floor=cfg.a_floor, dt_limit=cfg.dt_limit,
               rotation_range=cfg.rotation_range, b_norm_w=m.b_norm_w.cpu().numpy(),
               c_norm_w=m.c_norm_w.cpu().numpy(), b_bias=m.b_bias.cpu().numpy(), c_bias=m.c_bias.cpu().numpy(),
               D=m.D.cpu().numpy(), mimo_x=None if M == 1 else m.mimo_x.cpu().numpy(),
               mimo_z=None if M == 1 else m.mimo_z.cpu().numpy(), mimo_o=None if M == 1 else m.mimo_o.cpu().numpy())
    W, Wo = m.in_proj_w.cpu().numpy(), m.out_proj_w.cpu().numpy()
    c0 = _cache(0, b, prm, cfg.num_rope_angles, zero=True)
    proj = x.cpu().numpy() @ W
    r = oracle.mamba3_prep_fwd(proj, prm, c0)
    y, hT = oracle.ssd3(r["v"], r["da"], r["B"], r["C"], r["gamma"], r["scale"], r["h0"], chunk=8)
    want = oracle.mamba3_finish_fwd(y, r["v"], proj[:, :, :cfg.d_inner], prm) @ Wo
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-3, atol=1e-4)
    c1 = dict(ssm=hT, k_state=r["k_state"], v_state=r["v_state"], angle=r["angle"])
    y2, _ = oracle.mamba3_step(xt.cpu().numpy() @ W, prm, c1)
    np.testing.assert_allclose(out2.cpu().numpy(), y2 @ Wo, rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("dtype,M", [("f32", 1), ("f32", 4), ("bf16", 4)])
def test_mamba3_forward_double_equals_single(dtype, M):
    """Mamba3::forward with a double-ssd cache (forward_double_ssd: its gamma and
    beta SSD calls as one 2M-rank mamba_ssd3_double_fwd) equals the single-ssd
    pathway from the same cache (the reference's single == double relation):
    outputs and every cache tensor, over a prompt and then a continuation whose
    beta term starts from the cache's x_prev / K_prev.  bf16 runs the config-4
    head shape (P 64, N 128, MIMO 4) on the MFMA paths."""
    import torch
    import mamba_hip
    if dtype == "f32":
        cfg = mamba_hip.Mamba3Config(d_model=64, state_rank=32, per_head_dim=16, mimo_rank=M, rope_fraction=0.5)
        tdt, tol, stol = torch.float32, dict(rtol=1e-3, atol=1e-4), dict(rtol=1e-3, atol=1e-4)
    else:
        cfg = mamba_hip.Mamba3Config(d_model=128, state_rank=128, per_head_dim=64, mimo_rank=M)
        tdt, tol, stol = torch.bfloat16, dict(rtol=2e-2, atol=1e-2), dict(rtol=2e-2, atol=1e-2)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(40 + M)
    m = cfg.init("cuda", tdt, gen)
    m.b_bias.normal_(0, 0.1, generator=gen)
    m.D.normal_(0, 1, generator=gen)
    b = 2
    x1 = torch.randn((b, 150, cfg.d_model), generator=gen, device="cuda").to(tdt)
    x2 = torch.randn((b, 70, cfg.d_model), generator=gen, device="cuda").to(tdt)
    cs, cd = m.new_cache(b, "single"), m.new_cache(b, "double")
    outs = []
    for x in (x1, x2):
        o_s, cs = m.forward(x, cs, chunk_len=32)
        o_d, cd = m.forward(x, cd, chunk_len=32)
        outs.append((o_s, o_d))
    torch.cuda.synchronize()
    assert cs.pathway == "single" and cd.pathway == "double"
    for o_s, o_d in outs:
        np.testing.assert_allclose(o_d.float().cpu().numpy(), o_s.float().cpu().numpy(), **tol)
    for nm in ("ssm_bhpr", "k_state_bmhr", "v_state_bhp", "angle_bha"):
        np.testing.assert_allclose(getattr(cd, nm).cpu().numpy(), getattr(cs, nm).cpu().numpy(), **stol)


FAST_CASES = [
    # (b, L, H, P, G, N, M, rope_dim): proj rows padded to a multiple of 8 elements,
    # which selects the segment-parallel kernels (256-position segments)
    (2, 37, 4, 16, 2, 16, 1, 16),     # SISO, one segment
    (2, 300, 4, 16, 1, 32, 4, 32),    # MIMO 4, two segments
    (1, 700, 2, 8, 1, 16, 2, 8),      # partial rotation, three segments, ragged tail
    (2, 512, 4, 32, 2, 64, 1, 0),     # rotation off, exactly two segments
    (1, 270, 2, 8, 1, 8, 2, 8),       # dstate 8 with MIMO: both pair members in one thread
    # the benched config-4 instantiation (dstate 128: 16 threads per row, (k, k + 64)
    # partners by xor-8 lane exchange, the fixed (B/C, rank) mapping of MIMO 4),
    # full rotation, three segments with a ragged tail
    (1, 600, 8, 64, 1, 128, 4, 128),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", FAST_CASES)
def test_mamba3_prep_fwd_segments(case, dtype):
    """The segment-parallel prep (aligned proj rows): the angle carried across
    segments through the f64 segment totals, every output and the cache tail
    against the oracle."""
    import torch
    import mamba_hip
    import oracle
    b, L, H, P, G, N, M, R = case
    prm = _params(sum(case) + 5, H, P, G, N, M, R)
    cfg = _cfg(prm)
    A = cfg.num_rope_angles
    rng = np.random.default_rng(sum(case) + 6)
    proj = rng.standard_normal((b, L, cfg.d_in_proj)).astype(np.float32)
    pad = -(-cfg.d_in_proj // 8) * 8 + 8
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    wide = torch.zeros((b, L, pad), dtype=tdt, device="cuda")
    wide[:, :, :cfg.d_in_proj] = torch.from_numpy(proj).to(tdt).cuda()
    pin = wide[:, :, :cfg.d_in_proj]
    cache = _cache(sum(case) + 7, b, prm, A)
    cg = _gpu_cache(cache)
    a = mamba_hip.mamba3_prep_args(cfg, pin, cg, dt_bias=_g(prm, "dt_bias"), b_norm_w=_g(prm, "b_norm_w"),
                                   c_norm_w=_g(prm, "c_norm_w"), b_bias=_g(prm, "b_bias"),
                                   c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"))
    assert mamba_hip.mamba3_prep_fast_path(a) == 1
    out = mamba_hip.mamba3_prep_fwd(cfg, pin, cg, dt_bias=_g(prm, "dt_bias"), b_norm_w=_g(prm, "b_norm_w"),
                                    c_norm_w=_g(prm, "c_norm_w"), b_bias=_g(prm, "b_bias"),
                                    c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"))
    torch.cuda.synchronize()
    r = oracle.mamba3_prep_fwd(pin.float().cpu().numpy(), prm, cache)
    io_tol = dict(rtol=2e-2, atol=1e-2) if dtype == "bf16" else F32_TOL
    np.testing.assert_allclose(out["v"].float().cpu().numpy(), r["v"], **io_tol, err_msg="v")
    for k in ("B", "C"):
        # rotated rows: an angle error d moves each rotated pair by d times the
        # pair's length, so the f32 bar is relative to each row's scale (f32
        # angles carried over hundreds of positions err by ~1e-6 rad)
        got, want = out[k].float().cpu().numpy(), r[k]
        if dtype == "bf16":
            np.testing.assert_allclose(got, want, **io_tol, err_msg=k)
        else:
            row = np.abs(want).max(axis=-1, keepdims=True)
            bad = np.abs(got - want) > F32_TOL["atol"] + F32_TOL["rtol"] * row
            assert not bad.any(), f"{k}: {int(bad.sum())} elements beyond rtol 1e-4 of their row's scale"
    for k in ("da", "gamma", "scale", "h0"):
        np.testing.assert_allclose(out[k].cpu().numpy(), r[k], **F32_TOL, err_msg=k)
    # the cache tail's k_state is the last rotated B row (f32): the same row-relative bar
    got, want = cg.k_state_bmhr.cpu().numpy(), r["k_state"]
    row = np.abs(want).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - want) <= F32_TOL["atol"] + F32_TOL["rtol"] * row), "k_state"
    np.testing.assert_allclose(cg.v_state_bhp.cpu().numpy(), r["v_state"], **F32_TOL)
    ag = cg.angle_bha.cpu().numpy()
    np.testing.assert_allclose(np.cos(ag), np.cos(r["angle"]), atol=5e-5)
    np.testing.assert_allclose(np.sin(ag), np.sin(r["angle"]), atol=5e-5)
