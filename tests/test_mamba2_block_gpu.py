"""Mamba-2 full-block prefill (Mamba2::forward, src/mamba2/mamba2.rs:546-786):
mamba2_conv_fwd and mamba2_gated_rmsnorm (C ABI) vs the CPU oracle, and
Mamba2.forward (in_proj -> conv prologue -> mamba_ssd2_fwd -> gated norm ->
out_proj) vs the oracle composition and vs its own decode steps.  f32 at
rtol 1e-4 (2e-4 through the chunked SSD); bf16 at rtol 2e-2 / atol 1e-2."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=2e-5)
BF16_TOL = dict(rtol=2e-2, atol=1e-2)


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


CONV_CASES = [
    # (b, L, channels, K, H, row_pad): row_pad 0 keeps 8-aligned rows (vector path)
    (2, 150, 40, 4, 3, 0),    # three tiles, vector path
    (1, 3, 24, 4, 2, 0),      # L < K: the window mixes cache and inputs
    (2, 70, 13, 3, 5, 3),     # odd channels: scalar path
    (1, 65, 16, 1, 2, 0),     # kernel 1
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", CONV_CASES)
def test_mamba2_conv_fwd_matches_oracle(case, dtype):
    import torch
    import mamba_hip
    import oracle
    from mamba_hip import _lib
    b, L, c, K, H, pad = case
    rng = np.random.default_rng(sum(case) + (dtype == "bf16"))
    xo = 8  # xBC columns start here (8-aligned)
    row = xo + c + H + 5 + pad
    row += (-row) % 8 if pad == 0 else 0
    proj = rng.standard_normal((b, L, row)).astype(np.float32)
    w = (rng.standard_normal((c, K)) / 2).astype(np.float32)
    bias = (0.1 * rng.standard_normal(c)).astype(np.float32)
    st0 = rng.standard_normal((b, c, K)).astype(np.float32)
    dtb = rng.uniform(-3, 1, H).astype(np.float32)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    pj = _t(proj, tdt)
    st = _t(st0)
    xbc = torch.empty((b, L, c), device="cuda", dtype=tdt)
    dt = torch.empty((b, L, H), device="cuda")
    a = _lib.Mamba2ConvArgs()
    a.batch, a.seqlen, a.channels, a.kernel, a.nheads = b, L, c, K, H
    a.in_dtype = a.out_dtype = 1 if dtype == "bf16" else 0
    a.proj, a.proj_sb, a.proj_sl = pj.data_ptr(), pj.stride(0), pj.stride(1)
    a.xbc_offset, a.dt_offset = xo, xo + c
    wt, bt, dtbt = _t(w), _t(bias), _t(dtb)
    a.conv_w, a.conv_b, a.conv_state, a.dt_bias = wt.data_ptr(), bt.data_ptr(), st.data_ptr(), dtbt.data_ptr()
    a.dt_min, a.dt_max = 1e-4, 5.0
    a.xbc, a.xbc_sb, a.xbc_sl, a.dt = xbc.data_ptr(), xbc.stride(0), xbc.stride(1), dt.data_ptr()
    assert _lib.lib().mamba2_conv_fwd(ctypes.byref(a), None) == 0
    torch.cuda.synchronize()
    rx, rdt, rst = oracle.mamba2_conv_fwd(pj.float().cpu().numpy(), w, bias, st0, dtb, xo, xo + c, c, H,
                                          dt_limit=(1e-4, 5.0))
    tol = BF16_TOL if dtype == "bf16" else F32_TOL
    np.testing.assert_allclose(xbc.float().cpu().numpy(), rx, **tol)
    np.testing.assert_allclose(dt.cpu().numpy(), rdt, **F32_TOL)
    np.testing.assert_allclose(st.cpu().numpy(), rst, rtol=0, atol=0)


@pytest.mark.parametrize("before", [False, True])
@pytest.mark.parametrize("dtype,W", [("f32", 96), ("bf16", 5120), ("f32", 37), ("bf16", 1000), ("bf16", 3072),
                                     ("bf16", 37), ("bf16-f32out", 2048)])
def test_mamba2_gated_rmsnorm_matches_oracle(dtype, W, before):
    import torch
    import mamba_hip
    import oracle
    rng = np.random.default_rng(W + before)
    b, L = 2, 5
    y = rng.standard_normal((b, L, W)).astype(np.float32)
    zw = rng.standard_normal((b, L, W + 24)).astype(np.float32)  # z as a slice of a wider row
    gamma = rng.uniform(0.5, 1.5, W).astype(np.float32)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    yt, zt = _t(y, tdt), _t(zw, tdt)[:, :, 8:8 + W]
    # bf16 rows of 8-multiple width take the register-resident kernel, the rest the streaming one
    out = None if dtype != "bf16-f32out" else torch.empty((b, L, W), device="cuda")
    out = mamba_hip.mamba2_gated_rmsnorm(yt, zt, _t(gamma), norm_before_gate=before, out=out)
    torch.cuda.synchronize()
    want = oracle.mamba2_gated_rmsnorm(yt.float().cpu().numpy(), zt.float().cpu().numpy(), gamma,
                                       mamba_hip.div_eps(tdt), before)
    tol = {"f32": F32_TOL, "bf16": BF16_TOL, "bf16-f32out": F32_TOL}[dtype]
    np.testing.assert_allclose(out.float().cpu().numpy(), want, **tol)


def _model(cfg, seed, dtype):
    import torch
    g = torch.Generator()
    g.manual_seed(seed)
    m = cfg.init("cuda", dtype, g)
    # non-trivial norm weight, D and conv bias
    m.norm_w = torch.from_numpy(np.random.default_rng(seed).uniform(0.5, 1.5, cfg.d_inner).astype(np.float32)).cuda()
    m.d = torch.from_numpy(np.random.default_rng(seed + 1).standard_normal(cfg.nheads).astype(np.float32)).cuda()
    return m


def _oracle_forward(m, x, cs0, ss0, chunk, io_round=None):
    """Oracle composition: in_proj (f64) -> mamba2_block_fwd -> out_proj (f64).
    ``io_round`` rounds where the bf16 model stores a tensor: the in_proj
    output, the conv output, the SSD's y, the normed output and the block
    output."""
    import oracle
    rnd = io_round if io_round is not None else (lambda a: a)
    c = m.cfg
    proj = rnd(x.astype(np.float64) @ m.in_proj_w.float().cpu().numpy().astype(np.float64))
    p = dict(conv_w=m.conv_w.cpu().numpy(), conv_b=None if m.conv_b is None else m.conv_b.cpu().numpy(),
             dt_bias=m.dt_bias.cpu().numpy(), A=m.A.cpu().numpy(), D=m.d.cpu().numpy(),
             norm_w=m.norm_w.cpu().numpy())
    cfgd = dict(nheads=c.nheads, headdim=c.per_head_dim, ngroups=c.ngroups, dstate=c.state_rank,
                norm_before_gate=c.is_norm_before_gate, dt_limit=c.dt_limit)
    yn, cs, ss = oracle.mamba2_block_fwd(proj.astype(np.float32), p, cs0, ss0, chunk, cfgd,
                                         eps=2.0885676e-5 if io_round is not None else 8.1584695e-8,
                                         io_round=io_round)
    out = rnd(yn @ m.out_proj_w.float().cpu().numpy().astype(np.float64))
    return out, cs, ss


@pytest.mark.parametrize("G,before", [(1, False), (2, True)])
def test_mamba2_forward_f32_matches_oracle(G, before):
    """Mamba2.forward in f32 (the SSD's generic path) against the oracle
    composition, from a non-empty cache; outputs and both caches."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=64, state_rank=16, per_head_dim=16, ngroups=G, is_norm_before_gate=before)
    m = _model(cfg, 5 + G, torch.float32)
    b, L = 2, 37
    rng = np.random.default_rng(G)
    x = rng.standard_normal((b, L, cfg.d_model)).astype(np.float32)
    cs0 = rng.standard_normal((b, cfg.conv_dim, cfg.conv_kernel)).astype(np.float32)
    ss0 = (0.1 * rng.standard_normal((b, cfg.nheads, cfg.per_head_dim, cfg.state_rank))).astype(np.float32)
    cache = mamba_hip.Mamba2Cache(_t(cs0), _t(ss0))
    out, cache = m.forward(_t(x), cache, chunk_len=16)
    torch.cuda.synchronize()
    want, cs, ss = _oracle_forward(m, x, cs0, ss0, 16)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=2e-4, atol=2e-5)
    # the window holds in_proj outputs: the GPU GEMM and the f64 product differ by f32 rounding
    np.testing.assert_allclose(cache.conv_bvk.cpu().numpy(), cs, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), ss, rtol=2e-4, atol=2e-6)


def test_mamba2_forward_then_step():
    """Prefill a prompt with Mamba2.forward, then decode with Mamba2.step: every
    decoded token equals the same position of one forward over the whole
    sequence, and the caches agree (the conv window and state handover)."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=64, state_rank=16, per_head_dim=16, ngroups=2)
    m = _model(cfg, 21, torch.float32)
    b, L, extra = 2, 29, 4
    x = _t(np.random.default_rng(3).standard_normal((b, L + extra, cfg.d_model)).astype(np.float32))
    full, cfull = m.forward(x, None, chunk_len=16)
    _, cache = m.forward(x[:, :L].contiguous(), None, chunk_len=16)
    for t in range(extra):
        o, cache = m.step(x[:, L + t].contiguous(), cache)
        np.testing.assert_allclose(o.cpu().numpy(), full[:, L + t].cpu().numpy(), rtol=2e-4, atol=2e-5)
    torch.cuda.synchronize()
    np.testing.assert_allclose(cache.conv_bvk.cpu().numpy(), cfull.conv_bvk.cpu().numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), cfull.ssm_bhpr.cpu().numpy(), rtol=2e-4, atol=2e-6)


def test_mamba2_forward_bf16_config1_heads():
    """bf16 block at the config-1 head shape (P=64, N=128, 80 heads, d_model
    2560): the conv output feeds the MFMA SSD as strided group-form views."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=2560)
    m = _model(cfg, 9, torch.bfloat16)
    b, L = 1, 300
    rng = np.random.default_rng(9)
    x = rng.standard_normal((b, L, cfg.d_model)).astype(np.float32)
    xt = _t(x, torch.bfloat16)
    cache = m.new_cache(b)
    # the SSD inputs take the fast path
    out, cache = m.forward(xt, cache, chunk_len=256)
    torch.cuda.synchronize()
    proj = (xt.float() @ m.in_proj_w.float()).to(torch.bfloat16)
    xbc, dt = mamba_hip.mamba2_conv_fwd(cfg, proj, m.new_cache(b), m.conv_w, m.conv_b, m.dt_bias)
    di, N = cfg.d_inner, cfg.state_rank
    assert mamba_hip.ssd2_fast_path(xbc[:, :, :di].unflatten(2, (cfg.nheads, 64)), dt, m.A,
                                    xbc[:, :, di:di + N].unflatten(2, (1, N)), xbc[:, :, di + N:].unflatten(2, (1, N)),
                                    chunk_len=256)
    # the oracle rounds to bf16 where the bf16 model stores a tensor (in_proj,
    # conv and SSD outputs, normed values, block output), so the bars are
    # north_star's absolute ones
    want, _, ss = _oracle_forward(m, xt.float().cpu().numpy(), np.zeros((b, cfg.conv_dim, 4), np.float32),
                                  np.zeros((b, cfg.nheads, 64, N), np.float32), 256, io_round=_bf16)
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, want, **BF16_TOL)
    np.testing.assert_allclose(cache.ssm_bhpr.cpu().numpy(), ss, **BF16_TOL)


def _bf16(a):
    from inputs import bf16_round
    return bf16_round(np.asarray(a, np.float32)).astype(np.float64)
