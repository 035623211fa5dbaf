"""BASELINE.json configs[4] at full size (batch 4 x 8192 steps, 32 heads,
headdim 64, dstate 128, MIMO rank 4, every rotation pair in use) against the
CPU oracle, so that the launch grid the benchmark runs (256 workgroups, each
walking all 256 fused chunks of its sequence), the 8192-step angle carry and
the f32 state carried across the whole sequence are covered.

* mamba_ssd3_fwd (the single-SSD seam, MFMA path) on the benchmark's own
  inputs (bench.make_ssd3_inputs), every batch row against oracle.ssd3
  (single_ssd/ssd/serial.rs:56-268).
* mamba3_ssd_fused_fwd (the prologue fused into the scan) on raw bf16 in_proj
  rows for all 4 batch rows, as a chain: equal bit for bit to the segment prep
  followed by the seam scan; that scan against oracle.ssd3 on the prep's own
  bf16 values over one whole row (all 8192 steps, all 32 heads); the prep
  against oracle.mamba3_prep_fwd (single_ssd/single_ssd/mod.rs:86-262).

Bars: north_star's bf16-in / f32-accumulate ones, rtol 2e-2 / atol 1e-2 on
every output element; rtol 1e-2 / atol 5e-3 on the f32 final state."""

import numpy as np
import pytest

from inputs import bf16_round

pytestmark = pytest.mark.gpu

BF16_TOL = dict(rtol=2e-2, atol=1e-2)
STATE_TOL = dict(rtol=1e-2, atol=5e-3)
CFG4 = dict(batch=4, seqlen=8192, mimo=4, nheads=32, headdim=64, dstate=128, chunk=128)


def test_ssd3_config4_full_size():
    import torch
    import bench
    import mamba_hip
    import oracle
    cfg = CFG4
    print("ssd3 config 4 full size", cfg, flush=True)
    inp = bench.make_ssd3_inputs(cfg, torch.device("cuda:0"), seed=3)
    assert mamba_hip.ssd3_fast_path(inp["v"], inp["da"], inp["B"], inp["C"], inp["gamma"], inp["scale"],
                                    chunk_len=cfg["chunk"])
    y, hT = mamba_hip.ssd3_fwd(inp["v"], inp["da"], inp["B"], inp["C"], inp["gamma"], inp["scale"], None,
                               chunk_len=cfg["chunk"])
    torch.cuda.synchronize()
    for row in range(cfg["batch"]):
        r = slice(row, row + 1)
        cpu = {k: inp[k][r].float().cpu().numpy() for k in ("v", "B", "C", "da", "gamma", "scale")}
        yo, ho = oracle.ssd3(cpu["v"], cpu["da"], cpu["B"], cpu["C"], cpu["gamma"], cpu["scale"], None, chunk=128)
        print(f"  row {row}: max |y| {np.abs(yo).max():.3g}", flush=True)
        np.testing.assert_allclose(y[r].float().cpu().numpy(), yo, **BF16_TOL, err_msg=f"y row {row}")
        np.testing.assert_allclose(hT[r].cpu().numpy(), ho, **STATE_TOL, err_msg=f"state row {row}")


def test_mamba3_fused_config4_full_size():
    """The fused kernel on config 4, checked stage by stage on identical inputs:
    (1) with D = NULL it equals the segment prep followed by the seam scan bit
    for bit (outputs, final state, cache tail of every row); (2) with D, its
    output matches oracle.ssd3 + D v on the prep's own bf16 v / B / C and f32
    coefficients at north_star's absolute bars, every element of one whole
    batch row (the grid's last workgroups); (3) the prep matches
    oracle.mamba3_prep_fwd on that row: v exactly, B and C within one bf16 unit
    (after 8192 steps of the f32 angle recurrence a few tenths of a percent of
    the elements round to the neighbouring bf16 value of the f64 oracle's),
    coefficients and cache tail at f32 tolerances."""
    import torch
    from test_mamba3_fused_gpu import _run_fused, _run_prep_seam, check_prep_against_oracle, oracle_on_prep
    from test_mamba3_prefill_gpu import _cache, _cfg, _params
    b, L, H, G, M, R = 4, 8192, 32, 1, 4, 128
    print("fused config 4 full size", (b, L, H, G, M, R), flush=True)
    prm = _params(41, H, 64, G, 128, M, R)
    cfg = _cfg(prm)
    rng = np.random.default_rng(42)
    proj = torch.from_numpy(rng.standard_normal((b, L, cfg.d_in_proj), dtype=np.float32)).to(torch.bfloat16)
    cache = _cache(43, b, prm, cfg.num_rope_angles)
    y0, h0, c0 = _run_fused(prm, cfg, proj, cache, with_d=False)
    pr, ys, hs, cu = _run_prep_seam(prm, cfg, proj, cache)
    # (1) bit for bit
    assert torch.equal(y0, ys), f"fused != prep + seam at {int((y0 != ys).sum())} elements"
    assert torch.equal(h0, hs)
    for nm in ("k_state_bmhr", "v_state_bhp", "angle_bha"):
        assert torch.equal(getattr(c0, nm), getattr(cu, nm)), nm
    del y0, ys
    # (2) the product path (with D) against the oracle scan on the prep's values
    y, hT, cg = _run_fused(prm, cfg, proj, cache)
    assert torch.equal(hT, hs)
    row = b - 1
    sl = slice(row, row + 1)
    want, ho = oracle_on_prep(pr, prm, sl=sl)
    got = y[sl].float().cpu().numpy()
    print(f"  row {row}: max |y| {np.abs(want).max():.3g}, worst |err| / bar "
          f"{np.max(np.abs(got - want) / (1e-2 + 2e-2 * np.abs(want))):.3f}", flush=True)
    np.testing.assert_allclose(got, want, **BF16_TOL)
    np.testing.assert_allclose(hT[sl].cpu().numpy(), ho, **STATE_TOL)
    # (3) the prologue against the f64 oracle on that row
    fr = check_prep_against_oracle(pr, cu, proj, prm, cache, sl=sl)
    print("  B / C one unit from the oracle's rounding:", fr, flush=True)
