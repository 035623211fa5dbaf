"""The Mamba-3 prologue fused into the single-SSD scan (mamba3_ssd_fused_fwd,
C ABI) against the CPU oracle, oracle.mamba3_prep_fwd -> oracle.ssd3 plus the
D skip (single_ssd/single_ssd/mod.rs:86-290): y per rank, the final state and
the cache tail (last rotated B, last x, wrapped angle).  Cases: the config-4
head shape (headdim 64, dstate 128, MIMO 4, every pair rotated) over several
chunks with a ragged tail, MIMO 2 with two groups and half the pairs rotated,
MIMO 8 with the rotation off.  Also against the unfused GPU sequence
(mamba3_prep_fwd -> mamba_ssd3_fwd) on the same inputs, and the block forward
taking the fused path.  bf16 in_proj rows and y: outputs within rtol 2e-2 /
atol 1e-2 of the output scale."""

import numpy as np
import pytest

from test_mamba3_prefill_gpu import _cache, _cfg, _g, _gpu_cache, _params

pytestmark = pytest.mark.gpu

CASES = [
    # (b, L, H, G, M, rope_dim)
    (2, 100, 4, 1, 4, 128),   # config-4 head shape: 4 chunks of 32 steps, ragged tail
    (1, 257, 2, 1, 4, 128),   # one step past a chunk boundary
    (1, 70, 4, 2, 2, 64),     # MIMO 2 (64-step chunks), two groups, half the pairs rotated
    (2, 45, 2, 1, 8, 0),      # MIMO 8 (16-step chunks), rotation off
]


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


def _run_fused(prm, cfg, proj, cache):
    import torch
    import mamba_hip
    cg = _gpu_cache(cache)
    a = mamba_hip.mamba3_fused_args(cfg, _rows8(proj), cg, dt_bias=_g(prm, "dt_bias"), b_norm_w=_g(prm, "b_norm_w"),
                                    c_norm_w=_g(prm, "c_norm_w"), b_bias=_g(prm, "b_bias"),
                                    c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"), D=_g(prm, "D"))
    assert mamba_hip.mamba3_fused_supported(a) == 1
    y, hT = mamba_hip.mamba3_fused_run(a, cg)
    torch.cuda.synchronize()
    return y, hT, cg


def _close(got, want, rtol=2e-2, atol=1e-2):
    scale = float(np.abs(want).max())
    np.testing.assert_allclose(got / scale, want / scale, rtol=rtol, atol=atol)


@pytest.mark.parametrize("case", CASES)
def test_mamba3_fused_matches_oracle(case):
    import oracle
    print("fused vs oracle", case, flush=True)
    prm, cfg, proj, cache = _inputs(case)
    y, hT, cg = _run_fused(prm, cfg, proj, cache)
    r = oracle.mamba3_prep_fwd(proj.float().numpy(), prm, cache)
    yo, ho = oracle.ssd3(r["v"], r["da"], r["B"], r["C"], r["gamma"], r["scale"], r["h0"], chunk=32)
    want = yo + prm["D"][None, None, None, :, None] * r["v"]
    _close(y.float().cpu().numpy(), want)
    _close(hT.cpu().numpy(), ho)
    # the cache tail: last rotated B (f32), last x (exact), wrapped angle
    np.testing.assert_allclose(cg.k_state_bmhr.cpu().numpy(), r["k_state"], rtol=2e-3, atol=2e-3)
    np.testing.assert_array_equal(cg.v_state_bhp.cpu().numpy(), r["v_state"])
    ag = cg.angle_bha.cpu().numpy()
    np.testing.assert_allclose(np.cos(ag), np.cos(r["angle"]), atol=2e-4)
    np.testing.assert_allclose(np.sin(ag), np.sin(r["angle"]), atol=2e-4)


@pytest.mark.parametrize("case", CASES[:3])
def test_mamba3_fused_matches_unfused(case):
    """The same inputs through mamba3_prep_fwd -> mamba_ssd3_fwd (per-head v, B,
    C and coefficients in HBM) plus D v: the fused scan forms the same bf16
    operands in its loaders."""
    import torch
    import mamba_hip
    print("fused vs unfused", case, flush=True)
    prm, cfg, proj, cache = _inputs(case)
    y, hT, cg = _run_fused(prm, cfg, proj, cache)
    cu = _gpu_cache(cache)
    pr = mamba_hip.mamba3_prep_fwd(cfg, _rows8(proj), cu, dt_bias=_g(prm, "dt_bias"), b_norm_w=_g(prm, "b_norm_w"),
                                   c_norm_w=_g(prm, "c_norm_w"), b_bias=_g(prm, "b_bias"),
                                   c_bias=_g(prm, "c_bias"), mimo_x=_g(prm, "mimo_x"))
    yu, hu = mamba_hip.ssd3_fwd(pr["v"], pr["da"], pr["B"], pr["C"], pr["gamma"], pr["scale"], pr["h0"],
                                chunk_len=32)
    want = yu.float() + _g(prm, "D")[None, None, None, :, None] * pr["v"].float()
    torch.cuda.synchronize()
    _close(y.float().cpu().numpy(), want.cpu().numpy(), rtol=1e-2, atol=4e-3)
    _close(hT.cpu().numpy(), hu.cpu().numpy(), rtol=1e-2, atol=2e-3)
    np.testing.assert_allclose(cg.k_state_bmhr.cpu().numpy(), cu.k_state_bmhr.cpu().numpy(), rtol=2e-3, atol=2e-3)
    np.testing.assert_array_equal(cg.v_state_bhp.cpu().numpy(), cu.v_state_bhp.cpu().numpy())


def test_mamba3_fused_split_carries_cache():
    """Two fused calls (prompt, then continuation) equal one call over the
    concatenation: the final state, k_state / v_state and angle carry the
    sequence across calls through the beta seed."""
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
    _close(torch.cat([y1, y2], 1).float().cpu().numpy(), y.float().cpu().numpy(), rtol=1e-2, atol=4e-3)
    _close(h2.cpu().numpy(), hT.cpu().numpy(), rtol=1e-2, atol=2e-3)
    np.testing.assert_array_equal(c2.v_state_bhp.cpu().numpy(), cg.v_state_bhp.cpu().numpy())


def test_mamba3_block_forward_takes_fused_path():
    """Mamba3.forward (single-ssd cache) at the config-4 head shape runs the
    fused scan, and equals the same block through the unfused sequence."""
    import torch
    import mamba_hip
    from mamba_hip import mamba3 as m3mod
    print("block forward fused", flush=True)
    cfg = mamba_hip.Mamba3Config(d_model=128, state_rank=128, per_head_dim=64, mimo_rank=4)
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
    _close(out_f.float().cpu().numpy(), out_u.float().cpu().numpy(), rtol=2e-2, atol=2e-2)
    _close(cf.ssm_bhpr.cpu().numpy(), hu.cpu().numpy(), rtol=1e-2, atol=2e-3)
