"""Mamba-2 decode step: libmamba_hip.so (C ABI) vs the CPU oracle.

* mamba2_step_ssm (everything of Mamba2::step between in_proj and out_proj)
  against oracle.mamba2_step_ssm over several consecutive steps, so the conv
  window slide and the state recurrence are both exercised; f32 I/O at rtol
  1e-4, bf16 I/O at rtol 2e-2 / atol 1e-2.
* The pre-norm layer (RmsNorm -> in_proj -> step -> out_proj -> residual)
  against oracle.mamba2_layer_step, with f32 weights (tight) and bf16 weights.
* A stack captured in a HIP graph: every replay equals the eager step.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=1e-5)
BF16_TOL = dict(rtol=2e-2, atol=1e-2)


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def _bf16_round(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def _ssm_inputs(seed, b, H, P, G, N, K):
    rng = np.random.default_rng(seed)
    d_inner, conv_dim = H * P, H * P + 2 * G * N
    dt0 = np.exp(rng.uniform(np.log(1e-3), np.log(0.1), H))
    return dict(
        conv_w=rng.uniform(-0.5, 0.5, (conv_dim, K)).astype(np.float32),
        conv_b=rng.uniform(-0.5, 0.5, conv_dim).astype(np.float32),
        dt_bias=(dt0 + np.log(-np.expm1(-dt0))).astype(np.float32),
        A=-rng.uniform(1, 16, H).astype(np.float32),
        D=rng.standard_normal(H).astype(np.float32),
        norm_w=(1 + 0.1 * rng.standard_normal(d_inner)).astype(np.float32),
        conv=rng.standard_normal((b, conv_dim, K)).astype(np.float32),
        ssm=(0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32),
        zx=[rng.standard_normal((b, d_inner + conv_dim + H)).astype(np.float32) for _ in range(3)],
    )


SSM_CASES = [
    # (b, H, P, G, N, K, zx dtype, out dtype, norm_before_gate)
    (3, 8, 64, 1, 128, 4, "f32", "f32", 0),     # fast kernel, dstate 128 (config-3 head shape)
    (2, 6, 64, 2, 64, 4, "f32", "f32", 0),      # fast kernel, dstate 64, two groups
    (2, 4, 64, 1, 128, 4, "bf16", "bf16", 0),   # bf16 in_proj output and out
    (1, 4, 64, 2, 128, 4, "f32", "f32", 1),     # norm before gate
    (2, 5, 16, 1, 24, 3, "f32", "f32", 0),      # generic kernel (headdim 16, dstate 24, width 3)
    (2, 3, 8, 3, 6, 2, "bf16", "f32", 1),       # generic, per-head groups
    (1, 2, 64, 1, 128, 1, "f32", "f32", 0),     # conv width 1 (no history)
]


@pytest.mark.parametrize("case", SSM_CASES)
def test_step_ssm_matches_oracle(case):
    import torch
    import mamba_hip
    import oracle
    b, H, P, G, N, K, zxd, outd, nbg = case
    dts = {"f32": torch.float32, "bf16": torch.bfloat16}
    inp = _ssm_inputs(sum(case[:6]), b, H, P, G, N, K)
    cfg = mamba_hip.Mamba2Config(d_model=H * P // 2, state_rank=N, conv_kernel=K, per_head_dim=P, ngroups=G,
                                 is_norm_before_gate=bool(nbg))
    assert cfg.nheads == H
    cache = mamba_hip.Mamba2Cache(conv_bvk=_t(inp["conv"]), ssm_bhpr=_t(inp["ssm"]))
    out = torch.empty(b, H * P, device="cuda", dtype=dts[outd])
    ws = torch.empty(1 << 20, device="cuda", dtype=torch.uint8)
    ref_conv, ref_ssm = inp["conv"], inp["ssm"]
    tol = F32_TOL if outd == "f32" else BF16_TOL
    for step, zx in enumerate(inp["zx"]):
        zx_in = zx if zxd == "f32" else _bf16_round(zx)
        zx_dev = _t(zx_in, dts[zxd])
        args = mamba_hip.step_ssm_args(cfg, zx_dev, cache, _t(inp["conv_w"]), _t(inp["conv_b"]),
                                       _t(inp["dt_bias"]), _t(inp["A"]), _t(inp["D"]), _t(inp["norm_w"]), out)
        mamba_hip.step_ssm(args, ws)
        torch.cuda.synchronize()
        ref_out, ref_conv, ref_ssm = oracle.mamba2_step_ssm(
            zx_in, ref_conv, inp["conv_w"], inp["conv_b"], inp["dt_bias"], inp["A"], inp["D"], inp["norm_w"],
            ref_ssm, H, P, G, N, norm_before_gate=bool(nbg))
        print(f"step {step}: case {case}", flush=True)
        np.testing.assert_array_equal(cache.conv_bvk.cpu().numpy(), ref_conv)
        np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), ref_ssm, **F32_TOL)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref_out, **tol)


def test_step_ssm_without_optional_inputs():
    """conv_b, dt_bias and D absent (NULL in the C ABI)."""
    import torch
    import mamba_hip
    import oracle
    b, H, P, G, N, K = 2, 4, 64, 1, 128, 4
    inp = _ssm_inputs(77, b, H, P, G, N, K)
    cfg = mamba_hip.Mamba2Config(d_model=128, state_rank=N, per_head_dim=P)
    cache = mamba_hip.Mamba2Cache(conv_bvk=_t(inp["conv"]), ssm_bhpr=_t(inp["ssm"]))
    out = torch.empty(b, H * P, device="cuda")
    ws = torch.empty(1 << 20, device="cuda", dtype=torch.uint8)
    args = mamba_hip.step_ssm_args(cfg, _t(inp["zx"][0]), cache, _t(inp["conv_w"]), None, None, _t(inp["A"]),
                                   None, _t(inp["norm_w"]), out)
    mamba_hip.step_ssm(args, ws)
    torch.cuda.synchronize()
    ref_out, ref_conv, ref_ssm = oracle.mamba2_step_ssm(
        inp["zx"][0], inp["conv"], inp["conv_w"], None, np.zeros(H, np.float32), inp["A"], None, inp["norm_w"],
        inp["ssm"], H, P, G, N)
    np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), ref_ssm, **F32_TOL)
    np.testing.assert_allclose(out.cpu().numpy(), ref_out, **F32_TOL)


def test_step_ssm_dt_limit_clamp():
    """dt is clamped to dt_limit after softplus (mamba2.rs:924)."""
    import torch
    import mamba_hip
    import oracle
    b, H, P, G, N, K = 1, 4, 64, 1, 64, 4
    inp = _ssm_inputs(5, b, H, P, G, N, K)
    cfg = mamba_hip.Mamba2Config(d_model=128, state_rank=N, per_head_dim=P, dt_limit=(0.02, 0.05))
    cache = mamba_hip.Mamba2Cache(conv_bvk=_t(inp["conv"]), ssm_bhpr=_t(inp["ssm"]))
    out = torch.empty(b, H * P, device="cuda")
    ws = torch.empty(1 << 20, device="cuda", dtype=torch.uint8)
    zx = inp["zx"][0]
    zx[:, -H:] = np.array([-10.0, -1.0, 1.0, 25.0], np.float32)  # below, inside, above, softplus-linear
    args = mamba_hip.step_ssm_args(cfg, _t(zx), cache, _t(inp["conv_w"]), _t(inp["conv_b"]), _t(inp["dt_bias"]),
                                   _t(inp["A"]), _t(inp["D"]), _t(inp["norm_w"]), out)
    mamba_hip.step_ssm(args, ws)
    torch.cuda.synchronize()
    ref_out, _, ref_ssm = oracle.mamba2_step_ssm(
        zx, inp["conv"], inp["conv_w"], inp["conv_b"], inp["dt_bias"], inp["A"], inp["D"], inp["norm_w"],
        inp["ssm"], H, P, G, N, dt_limit=(0.02, 0.05))
    np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), ref_ssm, **F32_TOL)
    np.testing.assert_allclose(out.cpu().numpy(), ref_out, **F32_TOL)


def test_rmsnorm_residual():
    import torch
    import mamba_hip
    import oracle
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 2560)).astype(np.float32)
    add = rng.standard_normal((5, 2560)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2560)).astype(np.float32)
    xd, out = _t(x), torch.empty(5, 2560, device="cuda")
    mamba_hip.rmsnorm(xd, _t(w), out=out, add=_t(add))
    torch.cuda.synchronize()
    np.testing.assert_allclose(xd.cpu().numpy(), x + add, rtol=0, atol=0)
    np.testing.assert_allclose(out.cpu().numpy(), oracle.rmsnorm(x + add, w), **F32_TOL)
    outb = torch.empty(5, 2560, device="cuda", dtype=torch.bfloat16)
    mamba_hip.rmsnorm(xd, _t(w), out=outb)  # no add: x unchanged
    torch.cuda.synchronize()
    np.testing.assert_allclose(xd.cpu().numpy(), x + add, rtol=0, atol=0)
    np.testing.assert_allclose(outb.float().cpu().numpy(), oracle.rmsnorm(x + add, w), **BF16_TOL)


def _oracle_params(layer):
    m = layer.mixer
    f = lambda t: None if t is None else t.float().cpu().numpy()  # noqa: E731
    return dict(pre_norm_w=f(layer.norm_w), w_in=f(m.in_proj_w), conv_w=f(m.conv_w), conv_b=f(m.conv_b),
                dt_bias=f(m.dt_bias), A=f(m.A), D=f(m.d), norm_w=f(m.norm_w), w_out=f(m.out_proj_w))


def _cfg_dict(cfg):
    return dict(nheads=cfg.nheads, headdim=cfg.per_head_dim, ngroups=cfg.ngroups, dstate=cfg.state_rank)


@pytest.mark.parametrize("wdtype", ["f32", "bf16"])
def test_layer_steps_match_oracle(wdtype):
    """Two pre-norm layers stepped three tokens: RmsNorm -> in_proj -> SSM step
    -> gated norm -> out_proj -> residual, caches carried between tokens
    (torch.mm products around mamba2_step_ssm)."""
    import torch
    import mamba_hip
    import oracle
    dt = torch.float32 if wdtype == "f32" else torch.bfloat16
    cfg = mamba_hip.Mamba2Config(d_model=256, state_rank=128, per_head_dim=64)
    gen = torch.Generator().manual_seed(11)
    stack = mamba_hip.Mamba2Stack.init(cfg, 2, "cuda", dt, gen, fused=False)
    b = 3
    rng = np.random.default_rng(12)
    caches = stack.new_caches(b)
    ref_caches = []
    for c in caches:
        c.conv_bvk.copy_(_t(rng.standard_normal(tuple(c.conv_bvk.shape)).astype(np.float32)))
        c.ssm_bhpr.copy_(_t((0.1 * rng.standard_normal(tuple(c.ssm_bhpr.shape))).astype(np.float32)))
        ref_caches.append([c.conv_bvk.cpu().numpy(), c.ssm_bhpr.cpu().numpy()])
    params = [_oracle_params(l) for l in stack.layers]
    tol = F32_TOL if wdtype == "f32" else BF16_TOL
    for step in range(3):
        x = rng.standard_normal((b, cfg.d_model)).astype(np.float32)
        y, caches = stack.step(_t(x), caches)
        torch.cuda.synchronize()
        u = x
        for i, p in enumerate(params):
            u, ref_caches[i][0], ref_caches[i][1] = oracle.mamba2_layer_step(
                u, p, ref_caches[i][0], ref_caches[i][1], _cfg_dict(cfg))
        print(f"step {step} ({wdtype})", flush=True)
        np.testing.assert_allclose(y.cpu().numpy(), u, **tol)
        for i, c in enumerate(caches):
            if wdtype == "f32":
                np.testing.assert_allclose(c.conv_bvk.cpu().numpy(), ref_caches[i][0], **F32_TOL)
                np.testing.assert_allclose(c.ssm_bhpr.cpu().numpy(), ref_caches[i][1], **F32_TOL)
            else:  # states of a bf16 model: inputs carry bf16 rounding of in_proj
                np.testing.assert_allclose(c.ssm_bhpr.cpu().numpy(), ref_caches[i][1], **BF16_TOL)


def test_mamba2_step_signature():
    """Mamba2::step(input_bm, None) allocates a zero cache like mamba2.rs:838-846."""
    import torch
    import mamba_hip
    import oracle
    cfg = mamba_hip.Mamba2Config(d_model=128, state_rank=64, per_head_dim=64)
    m = cfg.init("cuda", torch.float32, torch.Generator().manual_seed(1))
    x = np.random.default_rng(2).standard_normal((2, 128)).astype(np.float32)
    out, cache = m.step(_t(x), None)
    torch.cuda.synchronize()
    zx = oracle.linear(x, m.in_proj_w.cpu().numpy())
    ref, _, ref_ssm = oracle.mamba2_step_ssm(
        zx, np.zeros((2, cfg.conv_dim, 4), np.float32), m.conv_w.cpu().numpy(), m.conv_b.cpu().numpy(),
        m.dt_bias.cpu().numpy(), m.A.cpu().numpy(), m.d.cpu().numpy(), m.norm_w.cpu().numpy(),
        np.zeros((2, cfg.nheads, 64, 64), np.float32), cfg.nheads, 64, 1, 64)
    np.testing.assert_allclose(out.cpu().numpy(), oracle.linear(ref, m.out_proj_w.cpu().numpy()), **F32_TOL)
    np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), ref_ssm, **F32_TOL)


@pytest.mark.parametrize("fused,b", [(False, 4), (True, 40), (True, 64)])
def test_stack_hip_graph_replays_equal_eager(fused, b):
    """Capture one stack step in a HIP graph; replay it several times with eager
    work in between and check every replay against the eager result (batch 64:
    the two-stream half-batch schedule, captured as two branches)."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=256, state_rank=128, per_head_dim=64)
    stack = mamba_hip.Mamba2Stack.init(cfg, 3, "cuda", torch.bfloat16, torch.Generator().manual_seed(4), fused=fused)
    rng = np.random.default_rng(5)
    base = stack.new_caches(b)
    for c in base:
        c.conv_bvk.copy_(_t(rng.standard_normal(tuple(c.conv_bvk.shape)).astype(np.float32)))
        c.ssm_bhpr.copy_(_t((0.1 * rng.standard_normal(tuple(c.ssm_bhpr.shape))).astype(np.float32)))
    x0 = _t(rng.standard_normal((b, cfg.d_model)).astype(np.float32))

    def clone(cs):
        return [mamba_hip.Mamba2Cache(c.conv_bvk.clone(), c.ssm_bhpr.clone()) for c in cs]

    eager_caches = clone(base)
    x_e = x0.clone()
    stack.step_(x_e, eager_caches)
    torch.cuda.synchronize()

    gcaches = clone(base)
    x_g = x0.clone()
    stack.buffers(b, x_g.device)  # allocate outside the capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm up the BLAS handles on the capture stream
        stack.step_(x_g.clone(), clone(base))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stack.step_(x_g, gcaches)
    for rep in range(3):
        x_g.copy_(x0)
        for dst, src in zip(gcaches, base):
            dst.conv_bvk.copy_(src.conv_bvk)
            dst.ssm_bhpr.copy_(src.ssm_bhpr)
        _ = (x0 * 2).sum().item()  # eager work and a sync between replays
        g.replay()
        torch.cuda.synchronize()
        print(f"replay {rep}", flush=True)
        np.testing.assert_array_equal(x_g.cpu().numpy(), x_e.cpu().numpy())
        for a, e in zip(gcaches, eager_caches):
            np.testing.assert_array_equal(a.ssm_bhpr.cpu().numpy(), e.ssm_bhpr.cpu().numpy())
            np.testing.assert_array_equal(a.conv_bvk.cpu().numpy(), e.conv_bvk.cpu().numpy())


def test_step_invalid_args_raise():
    import torch
    import mamba_hip
    from mamba_hip import _lib
    a = _lib.Mamba2StepArgs()
    a.batch, a.nheads, a.headdim, a.ngroups, a.dstate, a.conv_kernel = 1, 4, 64, 1, 128, 4
    ws = torch.empty(16, device="cuda", dtype=torch.uint8)
    rc = _lib.lib().mamba2_step_ssm(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), 16, None)
    assert rc == 1  # required pointers missing
    with pytest.raises(mamba_hip.MambaHipError):
        mamba_hip.rmsnorm(torch.zeros(2, 3, device="cuda", dtype=torch.float64), None)


# ------------------------------------------------------------- fused path --

LIN_CASES = [
    # (rows, d_in, d_out, x dtype, y dtype, bias[, extra columns of x's row stride])
    # bf16 x with 16-byte aligned rows is read in place, anything else packed first;
    # weights up to 16 MB take one k-split with 4 / 8 / 16 waves per workgroup, and
    # 2 or 4 column parts per 32-column tile when the tiles are few
    (1, 256, 1000, "f32", "f32", False),     # one row (lin_gemv, packed), masked last stage, ragged last tile, 4 parts
    (1, 2560, 2560, "bf16", "bf16", True),   # one row (lin_gemv, in place), 16 waves, stages of 5
    (2, 512, 160, "f32", "f32", False),      # two rows (the MFMA kernel), packed operand, 4 parts
    (3, 1024, 96, "bf16", "f32", True),      # MT 1, in place, 16 waves, two pipeline stages per wave, 4 parts
    (32, 2048, 1024, "bf16", "bf16", True),  # the Mamba-3 half-batch out_proj: 32 tiles x 16 waves x 2 parts
    (16, 2560, 2560, "bf16", "bf16", True),  # 16 waves, walks of 10 k-steps: two stages of 5
    (8, 1792, 1024, "bf16", "f32", False),   # walks of 7: stages of 4, the second with one masked k-step; 2 parts
    (40, 512, 320, "bf16", "bf16", False),   # MT 2, in place: rows 40..63 read past x's end (zero)
    (100, 2048, 64, "f32", "f32", True),     # MT 4
    (200, 4096, 200, "bf16", "f32", False),  # MT 8, in place, 8 waves per workgroup
    (256, 64, 33, "f32", "f32", True),       # full 256 rows, K smaller than one stage
    (64, 2048, 1024, "bf16", "bf16", False),  # the Mamba-3 out_proj shape: 32 tiles x 16 waves
    (1, 1024, 5280, "bf16", "bf16", True),   # the Mamba-3 in_proj shape at batch 1
    (5, 1024, 2048, "bf16", "f32", False, 8),  # strided rows read in place, 8 waves
    (7, 512, 160, "bf16", "f32", True, 3),   # rows not 16-byte aligned: packed first
    (64, 2560, 10576, "bf16", "f32", False),  # 54 MB weight: k-split partial planes, summed
]


@pytest.mark.parametrize("case", LIN_CASES)
def test_linear_fwd_matches_oracle(case):
    """mamba_linear_fwd (packed bf16 weight, bf16 operand, f32 accumulation)
    against the oracle's f64 product of the same bf16-rounded operands."""
    import torch
    import mamba_hip
    import oracle
    rows, d_in, d_out, xd, yd, has_b = case[:6]
    pad = case[6] if len(case) > 6 else 0
    dts = {"f32": torch.float32, "bf16": torch.bfloat16}
    rng = np.random.default_rng(rows + d_in)
    W = (rng.standard_normal((d_in, d_out)) / np.sqrt(d_in)).astype(np.float32)
    x = rng.standard_normal((rows, d_in)).astype(np.float32)
    bias = rng.standard_normal(d_out).astype(np.float32) if has_b else None
    Wd = _t(W, torch.bfloat16)
    packed = mamba_hip.pack_linear(Wd)
    xdev = _t(np.pad(x, ((0, 0), (0, pad))), dts[xd])[:, :d_in]
    y = torch.empty(rows, d_out, device="cuda", dtype=dts[yd])
    mamba_hip.linear(xdev, packed, d_out, None if bias is None else _t(bias), out=y)
    torch.cuda.synchronize()
    ref = oracle.linear(_bf16_round(x), Wd.float().cpu().numpy(), bias)
    scale = np.abs(ref).max()
    tol = dict(rtol=2e-3, atol=2e-3 * scale) if yd == "f32" else dict(rtol=1e-2, atol=1e-2 * scale)
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, **tol)


def _randomize_caches(caches, rng):
    refs = []
    for c in caches:
        c.conv_bvk.copy_(_t(rng.standard_normal(tuple(c.conv_bvk.shape)).astype(np.float32)))
        c.ssm_bhpr.copy_(_t((0.1 * rng.standard_normal(tuple(c.ssm_bhpr.shape))).astype(np.float32)))
        refs.append([c.conv_bvk.cpu().numpy(), c.ssm_bhpr.cpu().numpy()])
    return refs


@pytest.mark.parametrize("b,d_model,nbg", [(3, 256, 0), (40, 512, 0), (100, 256, 1), (200, 256, 0), (2, 2048, 0)])
def test_fused_layer_steps_match_oracle(b, d_model, nbg):
    """mamba2_layer_step (packed products, 1/rms and residual in the out_proj
    epilogue, B/C window slide as its side job) over two layers and two tokens
    against the oracle's pre-norm layer step on the same bf16 weights."""
    import torch
    import mamba_hip
    import oracle
    cfg = mamba_hip.Mamba2Config(d_model=d_model, state_rank=128, per_head_dim=64, is_norm_before_gate=bool(nbg))
    stack = mamba_hip.Mamba2Stack.init(cfg, 2, "cuda", torch.bfloat16, torch.Generator().manual_seed(b), fused=True)
    assert stack.fused
    rng = np.random.default_rng(b)
    caches = stack.new_caches(b)
    refs = _randomize_caches(caches, rng)
    params = [_oracle_params(l) for l in stack.layers]
    for step in range(2):
        x = rng.standard_normal((b, d_model)).astype(np.float32)
        y, caches = stack.step(_t(x), caches)
        torch.cuda.synchronize()
        u = x
        for i, p in enumerate(params):
            u, refs[i][0], refs[i][1] = oracle.mamba2_layer_step(u, p, refs[i][0], refs[i][1], _cfg_dict(cfg),
                                                                 ) if not nbg else _layer_step_nbg(u, p, refs[i], cfg)
        print(f"b={b} d_model={d_model} step {step}", flush=True)
        np.testing.assert_allclose(y.cpu().numpy(), u, **BF16_TOL)
        for i, c in enumerate(caches):
            np.testing.assert_allclose(c.conv_bvk.cpu().numpy(), refs[i][0], **BF16_TOL)
            np.testing.assert_allclose(c.ssm_bhpr.cpu().numpy(), refs[i][1], **BF16_TOL)


def _layer_step_nbg(u, p, ref, cfg):
    """oracle.mamba2_layer_step with norm_before_gate (composed from the same
    oracle pieces)."""
    import oracle
    normed = oracle.rmsnorm(u, p["pre_norm_w"])
    zx = oracle.linear(normed, p["w_in"])
    out, cs, ss = oracle.mamba2_step_ssm(zx, ref[0], p["conv_w"], p["conv_b"], p["dt_bias"], p["A"], p["D"],
                                         p["norm_w"], ref[1], cfg.nheads, cfg.per_head_dim, cfg.ngroups,
                                         cfg.state_rank, norm_before_gate=True)
    return u + oracle.linear(out, p["w_out"]), cs, ss


@pytest.mark.parametrize("b", [35, 36, 64, 100, 256])
def test_half_batch_schedule_matches_one_stream(b):
    """The fused stack at a batch of 34 to 256 runs as two row parts (halves) on
    two streams (35: 17 and 18 rows; 36: halves of 18 rows; 100: halves of 50
    rows, a ragged last row tile); the same stack
    with the schedule off (one mamba2_stack_step over all rows) gives the same
    outputs and caches. The half batches' products may tile rows and split K
    differently, so f32 sums round in another order, and now and then that flips
    the rounding of a bf16 operand the fused step writes (the pre-normed row,
    the gated values): one bf16 ulp (2^-8 relative) of one term, hence 5e-3."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=512, state_rank=128, per_head_dim=64)
    split = mamba_hip.Mamba2Stack.init(cfg, 2, "cuda", torch.bfloat16, torch.Generator().manual_seed(11))
    whole = mamba_hip.Mamba2Stack(split.layers, split_batch=False)
    assert split.splits(b) and not whole.splits(b)
    rng = np.random.default_rng(12)
    c1 = split.new_caches(b)
    _randomize_caches(c1, rng)
    c2 = [mamba_hip.Mamba2Cache(c.conv_bvk.clone(), c.ssm_bhpr.clone()) for c in c1]
    for _ in range(2):
        x = _t(rng.standard_normal((b, 512)).astype(np.float32))
        y1, c1 = split.step(x, c1)
        y2, c2 = whole.step(x, c2)
    torch.cuda.synchronize()
    tol = dict(rtol=5e-3, atol=5e-3)
    np.testing.assert_allclose(y1.cpu().numpy(), y2.cpu().numpy(), **tol)
    for a, e in zip(c1, c2):
        np.testing.assert_allclose(a.ssm_bhpr.cpu().numpy(), e.ssm_bhpr.cpu().numpy(), **tol)
        np.testing.assert_allclose(a.conv_bvk.cpu().numpy(), e.conv_bvk.cpu().numpy(), rtol=1e-2, atol=1e-2)


def test_fused_and_unfused_stacks_agree():
    """The fused layer step and the torch.mm + mamba2_step_ssm path compute the
    same function (bf16 weights)."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=512, state_rank=64, per_head_dim=64)
    fused = mamba_hip.Mamba2Stack.init(cfg, 3, "cuda", torch.bfloat16, torch.Generator().manual_seed(6))
    plain = mamba_hip.Mamba2Stack(fused.layers, fused=False)
    b = 16
    rng = np.random.default_rng(7)
    c1 = fused.new_caches(b)
    _randomize_caches(c1, rng)
    c2 = [mamba_hip.Mamba2Cache(c.conv_bvk.clone(), c.ssm_bhpr.clone()) for c in c1]
    for _ in range(3):
        x = _t(rng.standard_normal((b, 512)).astype(np.float32))
        y1, c1 = fused.step(x, c1)
        y2, c2 = plain.step(x, c2)
    torch.cuda.synchronize()
    # two bf16 approximations of the same f32 function (each within BF16_TOL of
    # the oracle, see above): their difference gets twice the absolute budget
    tol = dict(rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(y1.cpu().numpy(), y2.cpu().numpy(), **tol)
    for a, e in zip(c1, c2):
        np.testing.assert_allclose(a.ssm_bhpr.cpu().numpy(), e.ssm_bhpr.cpu().numpy(), **tol)
        # windows hold raw bf16 in_proj outputs: a different accumulation order can move them by one bf16 ulp
        np.testing.assert_allclose(a.conv_bvk.cpu().numpy(), e.conv_bvk.cpu().numpy(), **tol)


@pytest.mark.parametrize("b", [1, 16, 64, 256])
def test_fused_stack_config3_layer_shape(b):
    """BASELINE.json configs[3]'s layer shape at each of its batches (1, 16,
    64, 256): d_model 2560, 80 heads x 64, dstate 128, conv width 4, in_proj
    2560 -> 10576 and out_proj 5120 -> 2560 (the split-K products the
    benchmark runs; batches 64 and 256 step as two half batches on two
    streams).  Two fused layers step two tokens from random caches, against
    the oracle's pre-norm layer step (src/modules/layer.rs:224-228) on the same
    bf16 weights: outputs and both caches of every layer."""
    import torch
    import mamba_hip
    import oracle
    d_model = 2560
    cfg = mamba_hip.Mamba2Config(d_model=d_model)
    assert (cfg.nheads, cfg.d_in_proj, cfg.state_rank) == (80, 10576, 128)
    stack = mamba_hip.Mamba2Stack.init(cfg, 2, "cuda", torch.bfloat16, torch.Generator().manual_seed(64), fused=True)
    assert stack.fused
    rng = np.random.default_rng(64)
    caches = stack.new_caches(b)
    refs = _randomize_caches(caches, rng)
    params = [_oracle_params(l) for l in stack.layers]
    for step in range(2):
        x = rng.standard_normal((b, d_model)).astype(np.float32)
        y, caches = stack.step(_t(x), caches)
        torch.cuda.synchronize()
        u = x
        for i, p in enumerate(params):
            u, refs[i][0], refs[i][1] = oracle.mamba2_layer_step(u, p, refs[i][0], refs[i][1], _cfg_dict(cfg))
        print(f"config-3 layer shape, batch {b}, step {step}", flush=True)
        np.testing.assert_allclose(y.cpu().numpy(), u, **BF16_TOL)
        for i, c in enumerate(caches):
            np.testing.assert_allclose(c.conv_bvk.cpu().numpy(), refs[i][0], **BF16_TOL)
            np.testing.assert_allclose(c.ssm_bhpr.cpu().numpy(), refs[i][1], **BF16_TOL)


@pytest.mark.parametrize("cols,add_dt,out_dt,pad", [
    (1024, "bf16", "bf16", 0),   # register form, one float4 per thread: the Mamba-3 stack's norm
    (2560, "f32", "f32", 0),     # two float4 steps
    (3000, None, "bf16", 8),     # three steps, the last partial; strided rows (16-byte aligned)
    (4096, "bf16", "f32", 0),    # four steps
    (1000, "f32", "bf16", 0),    # register form with a 4000-byte row stride
    (1002, "bf16", "f32", 0),    # cols % 4 != 0: the scalar kernel
])
def test_rmsnorm_matches_oracle(cols, add_dt, out_dt, pad):
    """mamba_rmsnorm: x += add (in place, f32), out = RmsNorm(x) * w (rms_norm.rs:53-98)
    against the oracle's f64 RmsNorm of the same f32 sums; bf16 outputs within one bf16
    rounding, f32 within sum-order rounding."""
    import torch
    import mamba_hip
    import oracle
    rows = 7
    rng = np.random.default_rng(cols)
    dts = {"f32": torch.float32, "bf16": torch.bfloat16}
    x0 = rng.standard_normal((rows, cols)).astype(np.float32)
    w = (0.5 + rng.random(cols)).astype(np.float32)
    xd = torch.tensor(np.pad(x0, ((0, 0), (0, pad))), device="cuda")[:, :cols]
    add = None
    want_x = x0.copy()
    if add_dt is not None:
        a = rng.standard_normal((rows, cols)).astype(np.float32)
        add = torch.tensor(a, device="cuda").to(dts[add_dt])
        want_x = x0 + add.float().cpu().numpy()
    out = torch.empty((rows, cols + pad), device="cuda", dtype=dts[out_dt])[:, :cols]
    mamba_hip.step.rmsnorm(xd, torch.tensor(w, device="cuda"), out=out, add=add)
    torch.cuda.synchronize()
    np.testing.assert_allclose(xd.cpu().numpy(), want_x, rtol=1e-6, atol=1e-6)
    want = oracle.rmsnorm(want_x, w)
    got = out.float().cpu().numpy()
    if out_dt == "bf16":
        np.testing.assert_allclose(got, want, rtol=2 ** -8, atol=1e-6)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
