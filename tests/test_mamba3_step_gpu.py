"""Mamba-3 decode step: mamba3_step_ssm (C ABI) vs the CPU oracle
(oracle.mamba3_step: prep pinned by rotation/coefficient closed forms, the
state update pinned by unrolling against the chunked single-SSD oracle).
f32 at rtol 1e-4; bf16 output at rtol 2e-2 / atol 1e-2; every cache tensor
is checked after each step."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=2e-5)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _setup(seed, b, H, P, G, N, M, rope_frac, out_norm, proj_bf16=False):
    import mamba_hip
    rng = np.random.default_rng(seed)
    cfg = mamba_hip.Mamba3Config(d_model=H * P // 2, state_rank=N, per_head_dim=P, ngroups=G, mimo_rank=M,
                                 rope_fraction=rope_frac, has_outproj_norm=out_norm)
    A = cfg.num_rope_angles
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    prm = dict(nheads=H, headdim=P, ngroups=G, dstate=N, mimo=M, rope_dim=cfg.rope_dim,
               dt_bias=rng.uniform(-3, -1, H).astype(np.float32), a_floor=1e-4, dt_limit=(0.0, 65504.0),
               rotation_range=2.0, b_norm_w=rng.uniform(0.5, 1.5, N).astype(np.float32),
               c_norm_w=rng.uniform(0.5, 1.5, N).astype(np.float32), b_bias=0.1 * f(H, M, N),
               c_bias=0.1 * f(H, M, N), D=f(H),
               mimo_x=f(H, M, P) if M > 1 else None, mimo_z=f(H, M, P) if M > 1 else None,
               mimo_o=f(H, M, P) if M > 1 else None,
               out_norm_w=rng.uniform(0.5, 1.5, P).astype(np.float32) if out_norm else None)
    cache = dict(ssm=0.1 * f(b, H, P, N), k_state=(f(b, M, H, N) / np.sqrt(N)).astype(np.float32), v_state=f(b, H, P),
                 angle=rng.uniform(-3, 3, (b, H, A)).astype(np.float32))
    proj = f(b, cfg.d_in_proj)
    if proj_bf16:
        import torch
        proj = torch.from_numpy(proj).to(torch.bfloat16).float().numpy()
    return cfg, prm, cache, proj


def _run_gpu(cfg, prm, cache_g, proj, out_dtype=None, proj_bf16=False):
    import torch
    import mamba_hip
    pj = _t(proj).to(torch.bfloat16) if proj_bf16 else _t(proj)
    out = torch.empty((proj.shape[0], cfg.d_inner), device="cuda", dtype=out_dtype or torch.float32)
    g = lambda k: None if prm.get(k) is None else _t(prm[k])  # noqa: E731
    args = mamba_hip.mamba3_step_ssm_args(cfg, pj, cache_g, dt_bias=g("dt_bias"), b_norm_w=g("b_norm_w"),
                                          c_norm_w=g("c_norm_w"), b_bias=g("b_bias"), c_bias=g("c_bias"),
                                          D=g("D"), mimo_x=g("mimo_x"), mimo_z=g("mimo_z"),
                                          mimo_o=g("mimo_o"), out_norm_w=g("out_norm_w"), out=out)
    mamba_hip.mamba3_step_ssm(args, torch.device("cuda"))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _gpu_cache(cache):
    import mamba_hip
    return mamba_hip.Mamba3Cache(_t(cache["ssm"]), _t(cache["k_state"]), _t(cache["v_state"]), _t(cache["angle"]))


def _check_cache(cg, cr, tol):
    np.testing.assert_allclose(cg.ssm_bhpr.cpu().numpy(), cr["ssm"], **tol)
    np.testing.assert_allclose(cg.k_state_bmhr.cpu().numpy(), cr["k_state"], **tol)
    np.testing.assert_allclose(cg.v_state_bhp.cpu().numpy(), cr["v_state"], **tol)
    # angles: compare on the circle (both are wrapped to [-pi, pi])
    ag, ar = cg.angle_bha.cpu().numpy(), cr["angle"]
    np.testing.assert_allclose(np.cos(ag), np.cos(ar), atol=2e-5)
    np.testing.assert_allclose(np.sin(ag), np.sin(ar), atol=2e-5)


CASES = [
    # (b, H, P, G, N, M, rope_frac, out_norm)
    (3, 4, 16, 2, 16, 1, 1.0, False),   # SISO, pairwise rotation of every pair
    (2, 4, 16, 1, 32, 4, 1.0, False),   # MIMO 4, half-and-half rotation
    (2, 2, 8, 1, 8, 2, 0.5, True),      # partial rotation, gated norm
    (2, 4, 32, 2, 64, 1, 0.0, True),    # rotation off (angle still advances)
    (2, 4, 64, 1, 128, 4, 1.0, False),  # config-4 head shape
    (2, 4, 64, 2, 128, 1, 1.0, True),   # dstate 128 SISO pairs, two groups, gated norm
    (3, 4, 64, 1, 128, 2, 0.5, True),   # dstate 128 MIMO 2, partial rotation, gated norm
    (2, 2, 32, 1, 256, 8, 0.5, False),  # dstate 256: two rotation pairs per lane, MIMO 8
]


@pytest.mark.parametrize("case", CASES)
def test_mamba3_step_matches_oracle(case):
    import oracle
    cfg, prm, cache, proj = _setup(sum(int(v * 10) for v in case), *case)
    cg = _gpu_cache(cache)
    y = _run_gpu(cfg, prm, cg, proj)
    yr, cr = oracle.mamba3_step(proj, prm, cache)
    np.testing.assert_allclose(y, yr, **F32_TOL)
    _check_cache(cg, cr, F32_TOL)


def test_mamba3_step_bf16_proj_and_out():
    """bf16 in_proj row in, bf16 y out (the bf16 model), config-4 head shape."""
    import torch
    import oracle
    cfg, prm, cache, proj = _setup(17, 2, 4, 64, 1, 128, 4, 1.0, False, proj_bf16=True)
    cg = _gpu_cache(cache)
    y = _run_gpu(cfg, prm, cg, proj, out_dtype=torch.bfloat16, proj_bf16=True)
    yr, cr = oracle.mamba3_step(proj, prm, cache)
    np.testing.assert_allclose(y, yr, rtol=2e-2, atol=1e-2)
    _check_cache(cg, cr, F32_TOL)


def test_mamba3_step_unroll_carries_cache():
    """Six consecutive tokens through the GPU step equal six oracle steps
    carrying the oracle's cache."""
    import oracle
    cfg, prm, cache, _ = _setup(19, 2, 4, 16, 2, 32, 4, 0.5, True)
    rng = np.random.default_rng(23)
    cg = _gpu_cache(cache)
    cr = cache
    for _ in range(6):
        proj = rng.standard_normal((2, cfg.d_in_proj)).astype(np.float32)
        y = _run_gpu(cfg, prm, cg, proj)
        yr, cr = oracle.mamba3_step(proj, prm, cr)
        np.testing.assert_allclose(y, yr, rtol=2e-4, atol=5e-5)
    _check_cache(cg, cr, dict(rtol=2e-4, atol=5e-5))


def test_mamba3_block_step_and_fresh_cache():
    """Mamba3.step: in_proj -> mamba3_step_ssm -> out_proj from a fresh cache,
    against the oracle with the same (f32) products."""
    import torch
    import mamba_hip
    import oracle
    cfg = mamba_hip.Mamba3Config(d_model=64, state_rank=32, per_head_dim=16, mimo_rank=2)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    m = cfg.init("cuda", torch.float32, gen)
    x = torch.randn((3, 64), generator=gen, device="cuda")
    out, cache = m.step(x, None)
    out2, cache = m.step(x * 0.5, cache)
    torch.cuda.synchronize()
    prm = dict(nheads=cfg.nheads, headdim=16, ngroups=1, dstate=32, mimo=2, rope_dim=cfg.rope_dim,
               dt_bias=m.dt_bias.cpu().numpy(), a_floor=cfg.a_floor, dt_limit=cfg.dt_limit,
               rotation_range=cfg.rotation_range, b_norm_w=m.b_norm_w.cpu().numpy(),
               c_norm_w=m.c_norm_w.cpu().numpy(), b_bias=m.b_bias.cpu().numpy(), c_bias=m.c_bias.cpu().numpy(),
               D=m.D.cpu().numpy(), mimo_x=m.mimo_x.cpu().numpy(), mimo_z=m.mimo_z.cpu().numpy(),
               mimo_o=m.mimo_o.cpu().numpy())
    W, Wo = m.in_proj_w.cpu().numpy(), m.out_proj_w.cpu().numpy()
    c0 = {k: np.zeros(s, np.float32) for k, s in
          dict(ssm=(3, cfg.nheads, 16, 32), k_state=(3, 2, cfg.nheads, 32), v_state=(3, cfg.nheads, 16),
               angle=(3, cfg.nheads, cfg.num_rope_angles)).items()}
    xs = x.cpu().numpy()
    y1, c1 = oracle.mamba3_step(xs @ W, prm, c0)
    y2, _ = oracle.mamba3_step((xs * 0.5) @ W, prm, c1)
    np.testing.assert_allclose(out.cpu().numpy(), y1 @ Wo, rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(out2.cpu().numpy(), y2 @ Wo, rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("d_model,P,N,M,b,packed", [
    (128, 64, 128, 4, 3, True),     # config-4 head shape, MT 1 product tiles
    (128, 64, 128, 4, 40, True),    # MT 2
    (128, 64, 128, 4, 130, True),   # MT 8
    (40, 16, 32, 2, 5, False),      # d_model 40: not a multiple of 16, the library GEMM
])
def test_mamba3_block_step_bf16(d_model, P, N, M, b, packed):
    """Mamba3.step on a bf16 block, two steps from a fresh cache, against the
    oracle with the same bf16 weight values.  in_proj and out_proj run on the
    packed streaming product (mamba_linear_fwd) where its shape rules allow,
    else on the library GEMM; both round their outputs to bf16 as the bf16
    model stores them, which the oracle repeats, so the bars are north_star's
    absolute ones."""
    import torch
    import mamba_hip
    import oracle
    from inputs import bf16_round
    cfg = mamba_hip.Mamba3Config(d_model=d_model, state_rank=N, per_head_dim=P, mimo_rank=M)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(13 + b)
    m = cfg.init("cuda", torch.bfloat16, gen)
    x = torch.randn((b, d_model), generator=gen, device="cuda").to(torch.bfloat16)
    assert mamba_hip.step_mm_ok(x, m.in_proj_w) == packed
    out, cache = m.step(x, None)
    out2, cache = m.step((x.float() * 0.5).to(torch.bfloat16), cache)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    f = lambda t: None if t is None else t.float().cpu().numpy()  # noqa: E731
    prm = dict(nheads=cfg.nheads, headdim=P, ngroups=1, dstate=N, mimo=M, rope_dim=cfg.rope_dim,
               dt_bias=f(m.dt_bias), a_floor=cfg.a_floor, dt_limit=cfg.dt_limit, rotation_range=cfg.rotation_range,
               b_norm_w=f(m.b_norm_w), c_norm_w=f(m.c_norm_w), b_bias=f(m.b_bias), c_bias=f(m.c_bias), D=f(m.D),
               mimo_x=f(m.mimo_x), mimo_z=f(m.mimo_z), mimo_o=f(m.mimo_o))
    W, Wo = f(m.in_proj_w), f(m.out_proj_w)
    c0 = {k: np.zeros(sh, np.float32) for k, sh in
          dict(ssm=(b, cfg.nheads, P, N), k_state=(b, M, cfg.nheads, N), v_state=(b, cfg.nheads, P),
               angle=(b, cfg.nheads, cfg.num_rope_angles)).items()}
    xs = f(x)
    y1, c1 = oracle.mamba3_step(bf16_round(xs @ W), prm, c0)
    y2, _ = oracle.mamba3_step(bf16_round(f((x.float() * 0.5).to(torch.bfloat16)) @ W), prm, c1)
    for got, y in ((out, y1), (out2, y2)):
        want = bf16_round(bf16_round(y) @ Wo)
        np.testing.assert_allclose(f(got), want, rtol=2e-2, atol=1e-2)


def test_mamba3_step_validation():
    import torch
    import mamba_hip
    cfg, prm, cache, proj = _setup(29, 1, 2, 8, 1, 12, 1, 1.0, False)  # dstate 12 unsupported
    with pytest.raises(mamba_hip.MambaHipError, match="dstate"):
        _run_gpu(cfg, prm, _gpu_cache(cache), proj)
    cfg, prm, cache, proj = _setup(31, 1, 2, 8, 1, 16, 2, 1.0, False)
    prm = dict(prm, mimo_o=None)
    with pytest.raises(mamba_hip.MambaHipError, match="mimo_o"):
        _run_gpu(cfg, prm, _gpu_cache(cache), proj)
    del torch


def _stack_reference(stack, x, caches):
    """Layers::step over the stack's layers from Mamba3.step and torch ops:
    x += block(RmsNorm(x) * w) per layer (layer.rs:224-232), f32 residual."""
    import torch
    x = x.clone()
    for layer, cache in zip(stack.layers, caches):
        # RmsNorm with div_eps(F32) (src/utils/mod.rs:59-65), as the stack's kernel
        xn = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 8.1584695e-8) * layer.norm_w
        out, _ = layer.mixer.step(xn.to(torch.bfloat16), cache)
        x = x + out.float()
    return x


@pytest.mark.parametrize("b", [3, 36, 100, 256])
def test_mamba3_stack_step(b):
    """Mamba3Stack.step_ (rmsnorm + packed products + mamba3_step_ssm per layer;
    at 36 rows two row parts on two streams, at 100 rows four parts of 25 rows
    on four, at 256 four parts of 64 rows, whose products take two row tiles)
    against the same layers stepped through Mamba3.step with torch's norm and
    residual, two tokens, caches carried; then the same stack with the schedule
    off agrees."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba3Config(d_model=256, state_rank=128, per_head_dim=64, mimo_rank=4)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(41 + b)
    stack = mamba_hip.Mamba3Stack.init(cfg, 3, "cuda", torch.bfloat16, gen)
    for layer in stack.layers:
        layer.norm_w.uniform_(0.5, 1.5, generator=gen)
    whole = mamba_hip.Mamba3Stack(stack.layers, split_batch=False)
    assert stack.parts(b) == {3: 1, 36: 2, 100: 4, 256: 4}[b] and not whole.splits(b)
    c_stack, c_ref, c_whole = stack.new_caches(b), stack.new_caches(b), stack.new_caches(b)
    eps = None
    for _ in range(2):
        x = torch.randn((b, cfg.d_model), generator=gen, device="cuda")
        got = x.clone()
        stack.step_(got, c_stack)
        alt = x.clone()
        whole.step_(alt, c_whole)
        want = _stack_reference(stack, x, c_ref)
        torch.cuda.synchronize()
        eps = torch.finfo(torch.bfloat16).eps
        np.testing.assert_allclose(got.cpu().numpy(), want.cpu().numpy(), rtol=2e-2, atol=1e-2)
        # the row parts may split the products' k sums differently: a bf16 operand
        # may round one ulp apart, 2^-7 at magnitudes up to 2, which also shows in
        # outputs near zero
        np.testing.assert_allclose(got.cpu().numpy(), alt.cpu().numpy(), rtol=4 * eps, atol=1e-2)
    for cs, cr in zip(c_stack, c_ref):
        np.testing.assert_allclose(cs.ssm_bhpr.cpu().numpy(), cr.ssm_bhpr.cpu().numpy(), rtol=2e-2, atol=1e-2)
        # the stack's fused norm and torch's round the pre-normed rows apart by a bf16
        # ulp here and there, and the row parts and the whole batch run in_proj on
        # different product plans, so a dt or rotation column may sit a few bf16 ulps
        # (2^-8 relative each) apart: that moves the increment dt range pi tanh(rot)
        # (dt range pi <= ~0.3 rad here) by about 1 % of itself, carried two steps
        np.testing.assert_allclose(cs.angle_bha.cpu().numpy(), cr.angle_bha.cpu().numpy(), rtol=1e-5, atol=5e-3)


@pytest.mark.parametrize("b", [3, 36, 100])
def test_mamba3_stack_hip_graph_replays_equal_eager(b):
    """Capture one Mamba3Stack step in a HIP graph (36 rows: two row parts on two
    streams, two branches; 100 rows: four parts, four branches); replay it
    several times with eager work in between and check every replay against
    the eager step, bit for bit."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba3Config(d_model=256, state_rank=128, per_head_dim=64, mimo_rank=4)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(61 + b)
    stack = mamba_hip.Mamba3Stack.init(cfg, 2, "cuda", torch.bfloat16, gen)
    base = stack.new_caches(b)
    for c in base:
        c.ssm_bhpr.normal_(0.0, 0.1, generator=gen)
        c.k_state_bmhr.normal_(0.0, 0.1, generator=gen)
        c.v_state_bhp.normal_(0.0, 1.0, generator=gen)
        c.angle_bha.uniform_(-3.0, 3.0, generator=gen)
    x0 = torch.randn((b, cfg.d_model), generator=gen, device="cuda")
    names = ("ssm_bhpr", "k_state_bmhr", "v_state_bhp", "angle_bha")

    def clone(cs):
        return [mamba_hip.Mamba3Cache(*(getattr(c, n).clone() for n in names), c.pathway) for c in cs]

    eager = clone(base)
    x_e = x0.clone()
    stack.step_(x_e, eager)
    torch.cuda.synchronize()
    gcaches = clone(base)
    x_g = x0.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # buffers, arguments and streams made outside the capture
        stack.step_(x_g.clone(), gcaches)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stack.step_(x_g, gcaches)
    for rep in range(3):
        x_g.copy_(x0)
        for dst, src in zip(gcaches, base):
            for n in names:
                getattr(dst, n).copy_(getattr(src, n))
        _ = (x0 * 2).sum().item()  # eager work and a sync between replays
        g.replay()
        torch.cuda.synchronize()
        print(f"replay {rep}", flush=True)
        assert torch.equal(x_g, x_e)
        for a, e in zip(gcaches, eager):
            for n in names:
                assert torch.equal(getattr(a, n), getattr(e, n)), n
