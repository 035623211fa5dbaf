"""Mamba-1 block forward (Mamba1::forward, src/mamba1/mamba1.rs:278-352) on the
GPU: in_proj / x_proj / dt_proj / out_proj on the ROCm BLAS, the prefill conv
on mamba2_conv_fwd (no dt heads), the scan on mamba1_scan_fwd with bias,
softplus, D and the silu(res) gate fused.  Against oracle.mamba1_block_fwd
(pinned by forward == step unroll and split == full in test_oracle.py), then
continued by Mamba1.step against oracle.mamba1_block_step.  f32: rtol 1e-4
atol 1e-5; caches compared in every case."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-4, atol=1e-5)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _oracle_params(m):
    f = lambda t: None if t is None else t.float().cpu().numpy()  # noqa: E731
    return dict(in_proj_w=f(m.in_proj_w), conv_w=f(m.conv_w), conv_b=f(m.conv_b), x_proj_w=f(m.x_proj_w),
                dt_proj_w=f(m.dt_proj_w), dt_proj_b=f(m.dt_proj_b), A=f(m.A), D=f(m.d), out_proj_w=f(m.out_proj_w))


def _model(d_model, n, k, expand, dt_rank, seed):
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba1Config(d_model=d_model, state_rank=n, conv_kernel=k, expand=expand, dt_rank_=dt_rank)
    return cfg, cfg.init("cuda", torch.Generator().manual_seed(seed))


def _cache(cfg, b, random, seed):
    rng = np.random.default_rng(seed)
    if not random:
        return (np.zeros((b, cfg.d_inner, cfg.conv_kernel), np.float32),
                np.zeros((b, cfg.d_inner, cfg.state_rank), np.float32))
    return (rng.standard_normal((b, cfg.d_inner, cfg.conv_kernel)).astype(np.float32),
            rng.standard_normal((b, cfg.d_inner, cfg.state_rank)).astype(np.float32))


# (d_model, state_rank, conv_kernel, expand, dt_rank, batch, seqlen): the
# reference test configs at a longer sequence, a sequence shorter than the
# kernel, and a wider block with a ragged channel count
CASES = [(32, 8, 4, 2, None, 2, 37), (32, 16, 4, 2, None, 2, 64), (32, 8, 2, 2, None, 3, 21),
         (32, 8, 4, 1, None, 2, 40), (32, 8, 4, 2, 8, 2, 33), (48, 16, 4, 2, None, 1, 3),
         (200, 16, 4, 2, None, 2, 300)]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("random_init", [False, True])
def test_mamba1_forward_matches_oracle(case, random_init):
    import torch
    import mamba_hip
    import oracle
    dm, n, k, ex, r, b, L = case
    cfg, m = _model(dm, n, k, ex, r, seed=L)
    p = _oracle_params(m)
    x = np.random.default_rng(L + 1).standard_normal((b, L, dm)).astype(np.float32)
    conv0, ssm0 = _cache(cfg, b, random_init, seed=L + 2)
    cache = mamba_hip.Mamba1Cache(conv_bik=_t(conv0), ssm_bir=_t(ssm0))
    print(f"case {case} random_init={random_init}", flush=True)
    y, cache2 = m.forward(_t(x), cache)
    torch.cuda.synchronize()
    assert cache2 is cache
    yr, cr, sr = oracle.mamba1_block_fwd(x, p, conv0, ssm0)
    np.testing.assert_allclose(cache.conv_bik.cpu().numpy(), cr, **TOL)
    np.testing.assert_allclose(cache.ssm_bir.cpu().numpy(), sr, **TOL)
    np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)


def test_mamba1_forward_then_step_matches_oracle():
    """Prefill with forward, then decode with step from the returned cache."""
    import torch
    import oracle
    cfg, m = _model(64, 16, 4, 2, None, seed=11)
    p = _oracle_params(m)
    b, L = 2, 9
    rng = np.random.default_rng(12)
    x = rng.standard_normal((b, L, 64)).astype(np.float32)
    y, cache = m.forward(_t(x), None)
    torch.cuda.synchronize()
    yr, conv, ssm = oracle.mamba1_block_fwd(x, p, *_cache(cfg, b, False, 0))
    np.testing.assert_allclose(y.cpu().numpy(), yr, **TOL)
    for t in range(3):
        xt = rng.standard_normal((b, 64)).astype(np.float32)
        yt, cache = m.step(_t(xt), cache)
        torch.cuda.synchronize()
        ytr, conv, ssm = oracle.mamba1_block_step(xt, p, conv, ssm)
        print(f"step {t}", flush=True)
        np.testing.assert_allclose(cache.conv_bik.cpu().numpy(), conv, **TOL)
        np.testing.assert_allclose(cache.ssm_bir.cpu().numpy(), ssm, **TOL)
        np.testing.assert_allclose(yt.cpu().numpy(), ytr, **TOL)


def test_mamba1_forward_split_equals_full():
    """forward over a prefix then the suffix from the returned cache equals one
    forward (src/mamba1/mamba1/tests.rs:384-429), from a random cache."""
    import torch
    import mamba_hip
    cfg, m = _model(32, 8, 4, 2, None, seed=21)
    b, L, split = 2, 50, 13
    x = _t(np.random.default_rng(22).standard_normal((b, L, 32)).astype(np.float32))
    conv0, ssm0 = _cache(cfg, b, True, seed=23)
    full = mamba_hip.Mamba1Cache(conv_bik=_t(conv0), ssm_bir=_t(ssm0))
    part = mamba_hip.Mamba1Cache(conv_bik=_t(conv0), ssm_bir=_t(ssm0))
    y, _ = m.forward(x, full)
    ya, _ = m.forward(x[:, :split], part)
    yb, _ = m.forward(x[:, split:], part)
    torch.cuda.synchronize()
    np.testing.assert_allclose(torch.cat([ya, yb], 1).cpu().numpy(), y.cpu().numpy(), **TOL)
    np.testing.assert_allclose(part.conv_bik.cpu().numpy(), full.conv_bik.cpu().numpy(), **TOL)
    np.testing.assert_allclose(part.ssm_bir.cpu().numpy(), full.ssm_bir.cpu().numpy(), **TOL)


def test_mamba1_forward_rejects_empty_sequence():
    import mamba_hip
    _, m = _model(32, 8, 4, 2, None, seed=1)
    with pytest.raises(mamba_hip.MambaHipError):
        m.forward(_t(np.zeros((1, 0, 32), np.float32)))
