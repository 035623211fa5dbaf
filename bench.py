"""Benchmark of the MI355X SSM hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload ssd2]
                    [--no-cpu-baseline]

A "step" is one pass of the hot path over one batch of synthetic input that is
already resident in HBM.  The default workload is BASELINE.json configs[1]:
the Mamba-2 2.7B-shaped SSD prefill (batch 8 x 4096 tokens, 80 heads x 64,
d_state 128, one group, chunk 256, bf16 x/B/C/y, f32 dt/A/D and f32 state),
run through the C ABI (mamba_ssd2_fwd) exactly as a caller would.

Prints ONE JSON line.  `value` is whole-job tokens/s over K timed steps
(bracketed by torch.cuda.synchronize()).  `roofline` is computed for the
dominant kernel (the fused chunk-scan kernel): algorithmic HBM bytes of one
call divided by that kernel's mean duration, measured with HIP events recorded
by the library around that kernel on the launch stream.  `cpu_baseline` times
the CPU restatement of the reference algorithm (oracle/, f32, OpenMP) on a
bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "burn-mamba_amd"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, published
F32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense f32 MFMA, published

# The reference's benches warm up by time (criterion's warm-up of
# BENCH_TIME_MS / 5 = 1 s, benches/layer.rs:199-205) with an iteration floor
# on top (BENCH_WARMUP_ITERS, :189-198).  The same here: the W requested
# untimed steps are the floor, and untimed steps continue until the warm-up
# has kept the GPU busy for WARMUP_S seconds, so that a short step count
# still starts the timed region at the steady clock.
WARMUP_S = 1.0
_RAMP = {"steps": 0, "s": 0.0}


def warm(step, floor):
    """Run `floor` untimed steps, then more until WARMUP_S seconds have passed
    (synchronised); the totals go into the JSON line's warmup_ramp."""
    import torch
    t0 = time.perf_counter()
    n = 0
    for _ in range(floor):
        step()
        n += 1
    torch.cuda.synchronize()
    batch = 1
    while time.perf_counter() - t0 < WARMUP_S:
        for _ in range(batch):
            step()
        n += batch
        torch.cuda.synchronize()
        batch = min(batch * 2, 256)
    _RAMP["steps"] += n
    _RAMP["s"] += time.perf_counter() - t0
    log(f"warm-up: {n} untimed steps in {time.perf_counter() - t0:.2f} s")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------- workloads --

SSD2_CFG1 = dict(batch=8, seqlen=4096, nheads=80, headdim=64, dstate=128, ngroups=1, chunk=256)


def ssd2_algorithmic(cfg):
    """Compulsory HBM bytes and causal-exact FLOPs of one SSD forward:
    x, y bf16; dt f32; B, C bf16 (per group); final state f32 (zero initial
    state is not read); A, D f32.  FLOPs: per token H*(Q*P + 4*P*N) + G*Q*N."""
    b, l, h, p, n, g, q = (cfg[k] for k in ("batch", "seqlen", "nheads", "headdim", "dstate",
                                             "ngroups", "chunk"))
    tok = b * l
    bytes_ = tok * (h * p * (2 + 2) + h * 4 + 2 * g * n * 2) + b * h * p * n * 4 + 2 * h * 4
    flops = tok * (h * (q * p + 4 * p * n) + g * q * n)
    return bytes_, flops


def make_ssd2_inputs(cfg, dev, seed=0):
    """BASELINE.json configs[1] distributions, generated on the device:
    x~N(0,1); dt = softplus(N(0,1) + b_h) with b_h = softplus^-1(exp(U(ln1e-3, ln0.1)));
    A = -exp(U(ln1, ln16)); B, C ~ N(0,1)/sqrt(N); D ~ N(0,1)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    b, l, h, p, n, G = (cfg[k] for k in ("batch", "seqlen", "nheads", "headdim", "dstate", "ngroups"))
    x = torch.randn((b, l, h, p), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    dt_target = torch.exp(torch.empty(h, device=dev).uniform_(
        float(torch.log(torch.tensor(1e-3))), float(torch.log(torch.tensor(0.1))), generator=g))
    bias = dt_target + torch.log(-torch.expm1(-dt_target))
    dt = torch.nn.functional.softplus(torch.randn((b, l, h), generator=g, device=dev) + bias)
    A = -torch.exp(torch.empty(h, device=dev).uniform_(0.0, float(torch.log(torch.tensor(16.0))),
                                                       generator=g))
    Bm = (torch.randn((b, l, G, n), generator=g, device=dev) / n ** 0.5).to(torch.bfloat16)
    Cm = (torch.randn((b, l, G, n), generator=g, device=dev) / n ** 0.5).to(torch.bfloat16)
    D = torch.randn(h, generator=g, device=dev)
    return dict(x=x, dt=dt.contiguous(), A=A.contiguous(), B=Bm, C=Cm, D=D)


def cpu_baseline_ssd2(cfg, seed=0):
    """The f32 CPU restatement of the reference's serial K1-K5 SSD
    (oracle/, OpenMP over (batch, head)) on the whole workload (all
    sequences, full length, all heads): about 10 s on 16 host cores."""
    import numpy as np

    import oracle
    from inputs import ssd2_inputs
    oracle.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    inp = ssd2_inputs(seed, b=cfg["batch"], l=cfg["seqlen"], h=cfg["nheads"], p=cfg["headdim"],
                      g=cfg["ngroups"], n=cfg["dstate"])
    t0 = time.perf_counter()
    oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], None,
                chunk=cfg["chunk"], form="serial", prec=32)
    el = time.perf_counter() - t0
    del np
    return {"value": cfg["batch"] * cfg["seqlen"] / el, "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"the full workload ({cfg['batch']} x {cfg['seqlen']} tokens, {cfg['nheads']} heads), "
                      f"f32 serial K1-K5 restatement of the reference, {el:.2f} s"}


MAMBA1_CFG2 = dict(batch=8, dim=5120, seqlen=2048, dstate=16)


def mamba1_algorithmic(cfg):
    """Compulsory HBM bytes of one scan: u, delta, z read and y written (f32),
    B, C [b, n, l], A [d, n], D [d] read, final state [b, d, n] written; FLOPs
    ~ 6 per (token, state) (exp counted as one) + 4 per token."""
    b, d, l, n = (cfg[k] for k in ("batch", "dim", "seqlen", "dstate"))
    tok = b * l
    bytes_ = 4 * (4 * tok * d + 2 * tok * n + d * n + d + b * d * n)
    flops = tok * d * (6 * n + 4)
    return bytes_, flops


def make_mamba1_inputs(cfg, dev, seed=0):
    """u~N(0,1) [b,d,l]; delta = softplus(N(0,1)-4);
    A = -(1..n) per channel (S4D-real); B, C ~ N(0,1) [b,n,l]; D = 1; z~N(0,1)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    b, d, l, n = (cfg[k] for k in ("batch", "dim", "seqlen", "dstate"))
    u = torch.randn((b, d, l), generator=g, device=dev)
    delta = torch.nn.functional.softplus(torch.randn((b, d, l), generator=g, device=dev) - 4.0)
    A = -torch.arange(1, n + 1, device=dev, dtype=torch.float32).repeat(d, 1).contiguous()
    B = torch.randn((b, n, l), generator=g, device=dev)
    C = torch.randn((b, n, l), generator=g, device=dev)
    D = torch.ones(d, device=dev)
    z = torch.randn((b, d, l), generator=g, device=dev)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z)


def cpu_baseline_mamba1(cfg, seed=0):
    """The f32 CPU restatement of Mamba1::selective_scan's sequential loop
    (oracle/, OpenMP over (batch, channel)) on the whole workload."""
    import oracle
    from inputs import mamba1_inputs
    oracle.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    inp = mamba1_inputs(seed, b=cfg["batch"], d=cfg["dim"], l=cfg["seqlen"], n=cfg["dstate"])
    t0 = time.perf_counter()
    oracle.mamba1_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"], prec=32)
    el = time.perf_counter() - t0
    return {"value": cfg["batch"] * cfg["seqlen"] / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the full workload ({cfg['batch']} x {cfg['seqlen']} tokens, {cfg['dim']} channels), "
                      f"f32 sequential restatement of the reference loop, {el:.2f} s"}


def bench_mamba1(args):
    import torch

    import mamba_hip
    cfg = dict(MAMBA1_CFG2)
    dev = torch.device("cuda:0")
    inp = make_mamba1_inputs(cfg, dev)
    y = torch.empty_like(inp["u"])
    hT = torch.empty((cfg["batch"], cfg["dim"], cfg["dstate"]), device=dev)

    def step(events=None):
        mamba_hip.mamba1_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                              y=y, final_state=hT, events=events)

    ms_per_step, kern_ms = _time_steps(args, step)
    nbytes, flops = mamba1_algorithmic(cfg)
    tokens = cfg["batch"] * cfg["seqlen"]
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    return {
        "metric": "Mamba-1 selective scan tokens/s (2.8B layer, B=8 L=2048 D=5120 N=16) + % HBM roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (BASELINE.json configs[2] distributions, seed 0)",
        "config": {"workload": "mamba1_scan_cfg2", **cfg, "gate": "silu(z)", "entry": "mamba1_scan_fwd"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel_ms": kern_ms,
                     "algorithmic_bytes": nbytes},
    }


# The Mamba-1 block forward at the reference's own bench shape (benches/layer.rs:
# batch 2, sequence 256, d_model 256, state_rank 16 for Mamba-1, f32), whose
# median the reference publishes (bench.md:17), and at the config-2 layer shape.
MAMBA1_BLOCK_SHAPES = {
    "ref": dict(batch=2, seqlen=256, d_model=256, dstate=16),
    "cfg2": dict(batch=8, seqlen=2048, d_model=2560, dstate=16),
}
MAMBA1_BLOCK_PUBLISHED_MS = {"flex (CPU)": 71.78, "cuda": 23.36, "cuda + fusion + autotune": 40.56}


def bench_mamba1_block(args):
    """Mamba1::forward (src/mamba1/mamba1.rs:278-352) of one block from an
    empty cache: in_proj, the causal conv (mamba2_conv_fwd without dt heads),
    x_proj / dt_proj formed time-major, the selective scan (mamba1_scan_fwd
    with dt bias, softplus, D and the silu gate fused) and out_proj, f32 with
    reference-init weights.  `value` is tokens/s of the whole forward; the
    roofline is the scan kernel's (HIP events around it, every call)."""
    import torch

    import mamba_hip
    shp = dict(MAMBA1_BLOCK_SHAPES[args.m1_shape])
    dev = torch.device("cuda:0")
    cfg = mamba_hip.Mamba1Config(d_model=shp["d_model"], state_rank=shp["dstate"])
    m = cfg.init("cuda", torch.Generator(device=dev).manual_seed(0))
    x = torch.randn((shp["batch"], shp["seqlen"], shp["d_model"]), generator=torch.Generator(device=dev).manual_seed(1),
                    device=dev)

    def step(events=None):
        m.forward(x, None, events=events)

    ms_per_step, kern_ms = _time_steps(args, step)
    scan = dict(batch=shp["batch"], dim=cfg.d_inner, seqlen=shp["seqlen"], dstate=shp["dstate"])
    nbytes, _ = mamba1_algorithmic(scan)
    tokens = shp["batch"] * shp["seqlen"]
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    out = {
        "metric": f"Mamba-1 block forward tokens/s (B={shp['batch']} L={shp['seqlen']} d_model={shp['d_model']} "
                  f"N={shp['dstate']}, f32) + scan % HBM roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (x ~ N(0,1), reference init, seed 0)",
        "config": {"workload": f"mamba1_block_{args.m1_shape}", **shp, "d_inner": cfg.d_inner,
                   "dt_rank": cfg.dt_rank, "entry": "Mamba1.forward (products on rocBLAS, conv + scan here)"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel_ms": kern_ms,
                     "algorithmic_bytes": nbytes, "kernel": "mamba1 scan inside the block"},
    }
    if args.m1_shape == "ref":
        # published medians of this row on other hardware (the reference's own shape)
        out["reference_published_ms"] = dict(MAMBA1_BLOCK_PUBLISHED_MS, source="bench.md:17")
    return out


# The reference's own published rows (bench.md:17-45, criterion medians of one
# block at batch 2, sequence 256, d_model 256, state_rank 64 (16 for Mamba-1),
# per_head_dim 64, in the backend's default float, f32): forward and step.
REF_BLOCK_SHAPE = dict(batch=2, seqlen=256, d_model=256, state_rank=64, per_head_dim=64)
REF_BLOCK_PUBLISHED_MS = {
    ("forward", "mamba1"): ({"flex (CPU)": 71.78, "cuda": 23.36, "cuda + fusion + autotune": 40.56}, "bench.md:17"),
    ("forward", "mamba2"): ({"flex (CPU)": 23.79, "cuda": 1.80, "cuda + fusion + autotune": 2.11}, "bench.md:18"),
    ("forward", "mamba3/siso"): ({"flex (CPU)": 23.89, "cuda": 3.33, "cuda + fusion + autotune": 3.99}, "bench.md:19"),
    ("forward", "mamba3/mimo-rank4"): ({"flex (CPU)": 122.58, "cuda": 9.27, "cuda + fusion + autotune": 4.78},
                                       "bench.md:21"),
    ("forward", "mamba3/siso-double-ssd"): ({"flex (CPU)": 30.55, "cuda": 3.40, "cuda + fusion + autotune": 4.85},
                                            "bench.md:23"),
    ("step", "mamba1"): ({"flex (CPU)": 0.346, "cuda": 0.777, "cuda + fusion + autotune": 0.704}, "bench.md:41"),
    ("step", "mamba2"): ({"flex (CPU)": 0.296, "cuda": 0.738, "cuda + fusion + autotune": 0.933}, "bench.md:42"),
    ("step", "mamba3/siso"): ({"flex (CPU)": 0.337, "cuda": 1.46, "cuda + fusion + autotune": 1.97}, "bench.md:43"),
    ("step", "mamba3/mimo-rank4"): ({"flex (CPU)": 0.533, "cuda": 1.97, "cuda + fusion + autotune": 2.50},
                                    "bench.md:45"),
    ("step", "mamba3/siso-double-ssd"): ({"flex (CPU)": 0.321, "cuda": 1.46, "cuda + fusion + autotune": 1.99},
                                         "bench.md:47"),
}


def bench_ref_block(args):
    """One block at the reference's own bench shape and methodology
    (benches/layer.rs:89-101, 176-205, 293-395): f32 (the default float of the
    reference's backends), reference-init weights, input ~ N(0, 1); forward
    from an empty cache (a double-SSD cache for siso-double-ssd), or a decode
    step fed by the cache the previous step produced.  Every iteration is
    issued eagerly (no HIP graph) and the device is drained once per timed
    batch, as criterion's iter_custom does there.  `value` is ms per
    iteration; the line carries the reference's published medians of the same
    row (other hardware).  mimo-rank1 is the same block as siso here (the
    reference's siso_specialization switch changes its own kernels only)."""
    import torch

    import mamba_hip
    mode, case = args.ref_mode, args.ref_case
    shp = dict(REF_BLOCK_SHAPE)
    b, L, dm = shp["batch"], shp["seqlen"], shp["d_model"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    f32 = torch.float32
    if case == "mamba1":
        m = mamba_hip.Mamba1Config(d_model=dm, state_rank=16).init("cuda", gen)
    elif case == "mamba2":
        m = mamba_hip.Mamba2Config(d_model=dm, state_rank=shp["state_rank"],
                                   per_head_dim=shp["per_head_dim"]).init(dev, f32, gen)
    else:
        mimo = 4 if case == "mamba3/mimo-rank4" else 1
        m = mamba_hip.Mamba3Config(d_model=dm, state_rank=shp["state_rank"], per_head_dim=shp["per_head_dim"],
                                   mimo_rank=mimo).init(dev, f32, gen)
    double = case == "mamba3/siso-double-ssd"

    def fresh_cache():
        return m.new_cache(b, "double") if double else (m.new_cache(b) if mode == "step" else None)

    if mode == "forward":
        x = torch.randn((b, L, dm), generator=gen, device=dev)

        def it():
            m.forward(x, fresh_cache())
    else:
        x = torch.randn((b, dm), generator=gen, device=dev)
        state = {"cache": fresh_cache()}

        def it():
            _, state["cache"] = m.step(x, state["cache"])
    log(f"warmup {args.warmup}")
    warm(it, args.warmup)
    log(f"timing {args.steps} iterations")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        it()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    pub, src = REF_BLOCK_PUBLISHED_MS[(mode, case)]
    tokens = b * (L if mode == "forward" else 1)
    return {
        "metric": f"{case} block {mode} ms per iteration at the reference's bench shape (B={b} "
                  f"{'L=' + str(L) + ' ' if mode == 'forward' else ''}d_model={dm}, f32)",
        "value": ms, "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (x ~ N(0,1), reference init, seed 0)",
        "config": {"workload": f"ref_block_{mode}_{case.replace('/', '_')}", **shp,
                   "state_rank_used": 16 if case == "mamba1" else shp["state_rank"],
                   "tokens_per_s": tokens / (ms * 1e-3),
                   "timing": "eager iterations, one device drain per timed batch (as benches/layer.rs:176-187)"},
        "roofline": None,
        "reference_published_ms": dict(pub, source=src,
                                       note="criterion medians on unnamed CPU / NVIDIA hardware"),
    }


def cpu_baseline_mamba1_block(shape, budget_tokens=2048, seed=0):
    """oracle.mamba1_block_fwd (f32 C restatement, OpenMP) on one batch row of
    the same shape, at most `budget_tokens` tokens, scaled per token."""
    import numpy as np

    import oracle
    import torch
    import mamba_hip
    shp = dict(MAMBA1_BLOCK_SHAPES[shape])
    cfg = mamba_hip.Mamba1Config(d_model=shp["d_model"], state_rank=shp["dstate"])
    m = cfg.init("cpu", torch.Generator().manual_seed(seed))
    f = lambda t: None if t is None else t.float().numpy()  # noqa: E731
    p = dict(in_proj_w=f(m.in_proj_w), conv_w=f(m.conv_w), conv_b=f(m.conv_b), x_proj_w=f(m.x_proj_w),
             dt_proj_w=f(m.dt_proj_w), dt_proj_b=f(m.dt_proj_b), A=f(m.A), D=f(m.d), out_proj_w=f(m.out_proj_w))
    L = min(shp["seqlen"], budget_tokens)
    x = np.random.default_rng(seed).standard_normal((1, L, shp["d_model"])).astype(np.float32)
    cs = np.zeros((1, cfg.d_inner, cfg.conv_kernel), np.float32)
    ss = np.zeros((1, cfg.d_inner, cfg.state_rank), np.float32)
    t0 = time.perf_counter()
    oracle.mamba1_block_fwd(x, p, cs, ss, prec=32)
    el = time.perf_counter() - t0
    return {"value": L / el, "unit": "tokens/s", "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count())),
            "kind": "port", "sample": f"one batch row, {L} tokens, f32 restatement of Mamba1::forward ({el:.2f} s)"}


MAMBA1_STEP_CFG = dict(n_layers=64, dim=5120, dstate=16, conv_kernel=4)


def mamba1_step_algorithmic(cfg, batch):
    """Compulsory HBM bytes of one decode token through the SSM part of
    Mamba1::step (mamba1.rs:533-733) for every layer: conv window and state
    read + written (f32), x in, conv out, delta, z in, y out (f32), B and C,
    A, D, conv weight/bias.  Returns (all kernels, scan-step kernel) per step."""
    L, d, n, k = cfg["n_layers"], cfg["dim"], cfg["dstate"], cfg["conv_kernel"]
    conv = batch * d * k * 4 * 2 + batch * d * 4 * 2 + d * k * 4 + d * 4
    scan = batch * d * n * 4 * 2 + batch * d * 4 * 4 + batch * n * 4 * 2 + d * n * 4 + d * 4
    return L * (conv + scan), scan


def bench_mamba1_step(args):
    """64 layers of the Mamba-1 decode SSM step (conv window step + selective
    scan step) at the 2.8B layer shape, captured in one HIP graph; every layer
    owns its caches, so the states stream from HBM."""
    import torch

    import mamba_hip
    cfg = dict(MAMBA1_STEP_CFG)
    b = args.batch
    L, d, n, k = cfg["n_layers"], cfg["dim"], cfg["dstate"], cfg["conv_kernel"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    A = -torch.arange(1, n + 1, device=dev, dtype=torch.float32).repeat(d, 1).contiguous()
    D = torch.ones(d, device=dev)
    conv_w = torch.randn((d, k), generator=g, device=dev) / k ** 0.5
    conv_b = torch.randn(d, generator=g, device=dev) * 0.1
    states = [torch.randn((b, d, n), generator=g, device=dev) * 0.1 for _ in range(L)]
    convs = [torch.randn((b, d, k), generator=g, device=dev) for _ in range(L)]
    x = torch.randn((b, d), generator=g, device=dev)
    delta = torch.nn.functional.softplus(torch.randn((b, d), generator=g, device=dev) - 4.0)
    z = torch.randn((b, d), generator=g, device=dev)
    Bm = torch.randn((b, n), generator=g, device=dev)
    Cm = torch.randn((b, n), generator=g, device=dev)
    xc = torch.empty((b, d), device=dev)
    y = torch.empty((b, d), device=dev)

    def eager(events=None):
        for i in range(L):
            mamba_hip.conv1d_step(x, convs[i], conv_w, conv_b, silu=True, out=xc)
            mamba_hip.scan_step(xc, delta, A, Bm, Cm, states[i], D=D, z=z, y=y,
                                events=None if events is None else events[i])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eager()
    log(f"warmup {args.warmup}")
    warm(graph.replay, args.warmup)
    log(f"timing {args.steps} graph replays")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    pairs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(L)]
             for _ in range(args.steps)]
    for ev in pairs:
        eager(ev)
    torch.cuda.synchronize()
    durs = [a.elapsed_time(b_) for ev in pairs for a, b_ in ev]
    kern_ms = sum(durs) / len(durs)
    log(f"ms/step {ms_per_step:.4f}, scan-step kernel {kern_ms * 1e3:.2f} us (mean of {len(durs)})")
    step_bytes, kernel_bytes = mamba1_step_algorithmic(cfg, b)
    achieved = kernel_bytes / (kern_ms * 1e-3) / 1e9
    return {
        "metric": f"Mamba-1 decode SSM step us at batch {b} (64 layers, D=5120 N=16 K=4, 1 GPU) + % HBM roofline",
        "value": ms_per_step * 1e3, "unit": "us/step",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (config-2 shapes, states ~N(0,0.1), seed 0)",
        "config": {"workload": "mamba1_decode_step", **cfg, "batch": b, "graph": "hip graph of the 64-layer step",
                   "step_bytes": step_bytes, "step_hbm_gbs": step_bytes / (ms_per_step * 1e-3) / 1e9,
                   "entry": "mamba_conv1d_step + mamba1_scan_step per layer"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel_ms": kern_ms,
                     "algorithmic_bytes": kernel_bytes, "kernel": "mamba1_step_kernel (mean over all layers)"},
    }


def cpu_baseline_mamba1_step(cfg, batch, budget_s=10.0, seed=0):
    """oracle.conv1d_step + oracle.mamba1_step (f32 restatement) per layer,
    as many layers as fit in the budget, scaled to the 64-layer step."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(seed)
    d, n, k = cfg["dim"], cfg["dstate"], cfg["conv_kernel"]
    A = -np.tile(np.arange(1, n + 1, dtype=np.float32), (d, 1))
    D = np.ones(d, np.float32)
    w = (rng.standard_normal((d, k)) / k ** 0.5).astype(np.float32)
    bias = (0.1 * rng.standard_normal(d)).astype(np.float32)
    x = rng.standard_normal((batch, d)).astype(np.float32)
    delta = np.log1p(np.exp(rng.standard_normal((batch, d)) - 4.0)).astype(np.float32)
    z = rng.standard_normal((batch, d)).astype(np.float32)
    Bm = rng.standard_normal((batch, n)).astype(np.float32)
    Cm = rng.standard_normal((batch, n)).astype(np.float32)
    st = (0.1 * rng.standard_normal((batch, d, n))).astype(np.float32)
    cs = rng.standard_normal((batch, d, k)).astype(np.float32)
    done, t0 = 0, time.perf_counter()
    while done < cfg["n_layers"] and (done == 0 or time.perf_counter() - t0 < budget_s):
        xc, cs = oracle.conv1d_step(x, cs, w, bias, silu=True, prec=32)
        _, st = oracle.mamba1_step(xc, delta, A, Bm, Cm, st, D=D, z=z, prec=32)
        done += 1
    sec = (time.perf_counter() - t0) / done * cfg["n_layers"]
    return {"value": sec * 1e6, "unit": "us/step", "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count())),
            "kind": "port", "sample": f"{done} of {cfg['n_layers']} layers at batch {batch} ({sec * done / cfg['n_layers']:.1f} s), "
                                      "scaled to 64 layers; f32 conv-step + scan-step restatement"}


MAMBA3_STEP_CFG = dict(n_layers=64, d_model=1024, state_rank=128, per_head_dim=64, ngroups=1, mimo_rank=4)


def mamba3_step_algorithmic(cfg, batch):
    """Compulsory HBM bytes of one Mamba-3 decode token (Mamba3::step,
    double_ssd/double_ssd/mod.rs:634-760) per layer: in_proj/out_proj weights
    (bf16) once; the SSM kernel's cache read + written (state, K, v_state,
    angle; f32), its in_proj row in (bf16) and y out (bf16).
    Returns (step bytes, SSM-kernel bytes per launch)."""
    import mamba_hip
    c = mamba_hip.Mamba3Config(d_model=cfg["d_model"], state_rank=cfg["state_rank"],
                               per_head_dim=cfg["per_head_dim"], ngroups=cfg["ngroups"], mimo_rank=cfg["mimo_rank"])
    H, P, N, M, A = c.nheads, c.per_head_dim, c.state_rank, c.mimo_rank, c.num_rope_angles
    cache = batch * (H * P * N + M * H * N + H * P + H * A) * 4 * 2
    kern = cache + batch * c.d_in_proj * 2 + batch * c.d_inner * 2
    weights = (c.d_model * c.d_in_proj + c.d_inner * c.d_model) * 2
    step = cfg["n_layers"] * (weights + kern) + batch * c.d_model * 4 * 2
    return step, kern


def bench_mamba3_step(args):
    """64 Mamba-3 blocks stepping one token (in_proj -> mamba3_step_ssm ->
    out_proj, the products on the packed streaming kernel as Mamba3.step runs
    them), config-4 block shapes with the reference's init, every layer with its
    own weights and cache, captured in one HIP graph."""
    import torch

    import mamba_hip
    cfg = dict(MAMBA3_STEP_CFG)
    b = args.batch
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    c = mamba_hip.Mamba3Config(d_model=cfg["d_model"], state_rank=cfg["state_rank"],
                               per_head_dim=cfg["per_head_dim"], ngroups=cfg["ngroups"], mimo_rank=cfg["mimo_rank"])
    blocks = [c.init(dev, torch.bfloat16, gen) for _ in range(cfg["n_layers"])]
    caches = []
    for m in blocks:
        cc = m.new_cache(b)
        cc.ssm_bhpr.normal_(0.0, 0.1, generator=gen)
        cc.k_state_bmhr.normal_(0.0, 0.1, generator=gen)
        cc.v_state_bhp.normal_(0.0, 1.0, generator=gen)
        caches.append(cc)
    x0 = torch.randn((b, c.d_model), generator=gen, device=dev)

    def rows(lo, hi):
        """Buffers and step arguments of batch rows lo .. hi - 1 (cache slices)."""
        n = hi - lo
        projs = [torch.empty((n, c.d_in_proj), device=dev, dtype=torch.bfloat16) for _ in range(2)]
        ys = torch.empty((n, c.d_inner), device=dev, dtype=torch.bfloat16)
        xs = [torch.empty((n, c.d_model), device=dev, dtype=torch.bfloat16) for _ in range(2)]
        ws = torch.empty(8 << 20, device=dev, dtype=torch.uint8)  # product workspace, shared in order
        argl = []
        for i, m in enumerate(blocks):
            cc = caches[i]
            part = mamba_hip.Mamba3Cache(cc.ssm_bhpr[lo:hi], cc.k_state_bmhr[lo:hi], cc.v_state_bhp[lo:hi],
                                         cc.angle_bha[lo:hi], cc.pathway)
            argl.append(mamba_hip.mamba3_step_ssm_args(c, projs[i % 2], part, dt_bias=m.dt_bias,
                                                       b_norm_w=m.b_norm_w, c_norm_w=m.c_norm_w, b_bias=m.b_bias,
                                                       c_bias=m.c_bias, D=m.D, mimo_x=m.mimo_x, mimo_z=m.mimo_z,
                                                       mimo_o=m.mimo_o, out=ys))
        return lo, hi, projs, ys, xs, ws, argl

    # the host schedule of Mamba3Stack: a batch of 34 to 256 rows steps as row
    # parts of at most 32 rows on up to four streams (batch_parts), one part's
    # weight-streaming products beside another part's state kernel (rows never
    # interact; each part reads the weights once).  Per-layer kernel events
    # time the one-stream whole-batch step.
    K = 1 if getattr(args, "no_split", False) else mamba_hip.batch_parts(b, mamba_hip.Mamba3Stack.max_parts)
    split = K > 1
    whole = rows(0, b)
    bounds = [(b * k) // K for k in range(K + 1)]
    halves = [rows(bounds[k], bounds[k + 1]) for k in range(K)] if split else None
    streams = [torch.cuda.Stream() for _ in range(K)] if split else None

    def run(part, events=None):
        lo, hi, projs, ys, xs, ws, argl = part
        xs[0].copy_(x0[lo:hi])
        for i, m in enumerate(blocks):
            mamba_hip.step_mm(xs[0], m.in_proj_w, out=projs[i % 2], workspace=ws)
            mamba_hip.mamba3_step_ssm(argl[i], dev, None if events is None else events[i])
            mamba_hip.step_mm(ys, m.out_proj_w, out=xs[1], workspace=ws)

    if getattr(args, "m3_stack", False):
        # the library's stack: pre-norm residual layers (Layers::step), one
        # rmsnorm per layer on top of the blocks, the same schedule
        stack = mamba_hip.Mamba3Stack([mamba_hip.Mamba3Layer(torch.ones(c.d_model, device=dev), m) for m in blocks],
                                      split_batch=not getattr(args, "no_split", False))
        x_res = torch.empty((b, c.d_model), device=dev)
        stack.buffers(b, dev)

        def eager(events=None):
            x_res.copy_(x0)
            stack.step_(x_res, caches, events)
    else:
        eager = None

    # every block reads the same input row (no norm/residual between blocks
    # here, so chaining 64 of them would only grow or shrink the activations)
    def eager_blocks(events=None):
        if events is not None or not split:
            run(whole, events)
            return
        cur = torch.cuda.current_stream()
        for part, st in zip(halves, streams):
            st.wait_stream(cur)
            with torch.cuda.stream(st):
                run(part)
        for st in streams:
            cur.wait_stream(st)

    if eager is None:
        eager = eager_blocks
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eager()
    log(f"warmup {args.warmup}")
    warm(graph.replay, args.warmup)
    log(f"timing {args.steps} graph replays")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    L = cfg["n_layers"]
    pairs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(L)]
             for _ in range(args.steps)]
    for ev in pairs:
        eager(ev)
    torch.cuda.synchronize()
    durs = [a.elapsed_time(b_) for ev in pairs for a, b_ in ev]
    kern_ms = sum(durs) / len(durs)
    log(f"ms/step {ms_per_step:.4f}, SSM-step kernel {kern_ms * 1e3:.2f} us (mean of {len(durs)})")
    step_bytes, kernel_bytes = mamba3_step_algorithmic(cfg, b)
    achieved = kernel_bytes / (kern_ms * 1e-3) / 1e9
    return {
        "metric": f"Mamba-3 decode step us at batch {b} (64 layers, H=32 P=64 N=128 MIMO 4, 1 GPU) + % HBM roofline",
        "value": ms_per_step * 1e3, "unit": "us/step",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (config-4 block shapes, reference init, states ~N(0,0.1), seed 0)",
        "config": {"workload": "mamba3_decode_step", **cfg, "batch": b, "graph": "hip graph of the 64-layer step",
                   "step_bytes": step_bytes, "step_hbm_gbs": step_bytes / (ms_per_step * 1e-3) / 1e9,
                   "entry": "mamba_linear_fwd in_proj + mamba3_step_ssm + mamba_linear_fwd out_proj per layer",
                   "schedule": f"{K} row parts on {K} streams" if split else "one stream",
                   "layers": "Mamba3Stack: pre-norm residual layers (rmsnorm + block per layer)"
                   if getattr(args, "m3_stack", False) else "blocks (each reads the same input row)"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel_ms": kern_ms,
                     "algorithmic_bytes": kernel_bytes, "kernel": "mamba3_step_kernel (mean over all layers)"},
    }


def cpu_baseline_mamba3_step(cfg, batch, budget_s=10.0, seed=0):
    """oracle.mamba3_step (f32 restatement) plus numpy products per layer, as
    many layers as fit in the budget, scaled to the 64-layer step."""
    import numpy as np

    import mamba_hip
    import oracle
    rng = np.random.default_rng(seed)
    c = mamba_hip.Mamba3Config(d_model=cfg["d_model"], state_rank=cfg["state_rank"],
                               per_head_dim=cfg["per_head_dim"], ngroups=cfg["ngroups"], mimo_rank=cfg["mimo_rank"])
    H, P, N, M, A = c.nheads, c.per_head_dim, c.state_rank, c.mimo_rank, c.num_rope_angles
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    prm = dict(nheads=H, headdim=P, ngroups=c.ngroups, dstate=N, mimo=M, rope_dim=c.rope_dim,
               dt_bias=np.full(H, -2.0, np.float32), a_floor=c.a_floor, dt_limit=c.dt_limit,
               rotation_range=c.rotation_range, b_norm_w=np.ones(N, np.float32), c_norm_w=np.ones(N, np.float32),
               b_bias=np.ones((H, M, N), np.float32), c_bias=np.ones((H, M, N), np.float32),
               D=np.ones(H, np.float32), mimo_x=np.full((H, M, P), 1 / M, np.float32),
               mimo_z=np.ones((H, M, P), np.float32), mimo_o=np.full((H, M, P), 1 / M, np.float32))
    W = (f(c.d_model, c.d_in_proj) / np.sqrt(c.d_model)).astype(np.float32)
    Wo = (f(c.d_inner, c.d_model) / np.sqrt(c.d_inner)).astype(np.float32)
    cache = dict(ssm=0.1 * f(batch, H, P, N), k_state=0.1 * f(batch, M, H, N), v_state=f(batch, H, P),
                 angle=np.zeros((batch, H, A), np.float32))
    x = f(batch, c.d_model)
    done, t0 = 0, time.perf_counter()
    while done < cfg["n_layers"] and (done == 0 or time.perf_counter() - t0 < budget_s):
        y, cache = oracle.mamba3_step(x @ W, prm, cache, prec=32)
        _ = y @ Wo  # every block reads the same input row, as on the GPU
        done += 1
    sec = (time.perf_counter() - t0) / done * cfg["n_layers"]
    return {"value": sec * 1e6, "unit": "us/step", "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count())),
            "kind": "port", "sample": f"{done} of {cfg['n_layers']} layers at batch {batch} ({sec * done / cfg['n_layers']:.1f} s), "
                                      "scaled to 64 layers; f32 Mamba-3 step restatement + numpy products"}


def mamba3_prep_algorithmic(cfg):
    """Compulsory HBM bytes of one mamba3_prep_fwd call at config 4: the in_proj
    rows read (bf16), v / B / C written per head and rank (bf16), da / gamma /
    scale (f32), the initial state read + written (f32) and the small cache tail."""
    import mamba_hip
    c = mamba_hip.Mamba3Config(d_model=cfg["nheads"] * cfg["headdim"] // 2, state_rank=cfg["dstate"],
                               per_head_dim=cfg["headdim"], ngroups=1, mimo_rank=cfg["mimo"])
    b, L, H, P, N, M = cfg["batch"], cfg["seqlen"], c.nheads, c.per_head_dim, c.state_rank, c.mimo_rank
    tok = b * L
    return (tok * c.d_in_proj * 2 + tok * M * H * (P + 2 * N) * 2 + tok * H * 3 * 4 + 2 * b * H * P * N * 4
            + 2 * b * (M * H * N + H * P + H * c.num_rope_angles) * 4)


def bench_mamba3_prep(args):
    """mamba3_prep_fwd at config 4 (B=4 L=8192 H=32 P=64 N=128 MIMO 4, full
    rotation): the prologue from in_proj rows to the SSD seam's inputs."""
    import torch

    import mamba_hip
    cfg = dict(SSD3_CFG4)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    c = mamba_hip.Mamba3Config(d_model=cfg["nheads"] * cfg["headdim"] // 2, state_rank=cfg["dstate"],
                               per_head_dim=cfg["headdim"], ngroups=1, mimo_rank=cfg["mimo"])
    m = c.init(dev, torch.bfloat16, gen)
    b, L = cfg["batch"], cfg["seqlen"]
    proj = (torch.randn((b, L, c.d_in_proj), generator=gen, device=dev)).to(torch.bfloat16)
    cache = m.new_cache(b)

    def step():
        mamba_hip.mamba3_prep_fwd(c, proj, cache, dt_bias=m.dt_bias, b_norm_w=m.b_norm_w, c_norm_w=m.c_norm_w,
                                  b_bias=m.b_bias, c_bias=m.c_bias, mimo_x=m.mimo_x)

    log(f"warmup {args.warmup}")
    warm(step, args.warmup)
    log(f"timing {args.steps} steps")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    kern_ms = e0.elapsed_time(e1) / args.steps
    nbytes = mamba3_prep_algorithmic(cfg)
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    tokens = b * L
    return {
        "metric": "Mamba-3 prefill prologue tokens/s (B=4 L=8192 H=32 P=64 N=128 MIMO 4) + % HBM roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (config-4 shapes, reference init, in_proj rows ~N(0,1), seed 0)",
        "config": {"workload": "mamba3_prep_cfg4", **cfg, "io": "proj/v/B/C bf16, coefficients and states f32",
                   "entry": "mamba3_prep_fwd (seed, angle-total and segment prep kernels)"},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None, "kernel_ms": kern_ms,
                     "algorithmic_bytes": nbytes,
                     "timing": "HIP events around the back-to-back calls on the launch stream, per call"},
    }


def cpu_baseline_mamba3_prep(cfg, seed=0):
    """oracle.mamba3_prep_fwd (float64 numpy restatement) on one batch row's
    first 1024 tokens, scaled to the whole call."""
    import numpy as np

    import mamba_hip
    import oracle
    c = mamba_hip.Mamba3Config(d_model=cfg["nheads"] * cfg["headdim"] // 2, state_rank=cfg["dstate"],
                               per_head_dim=cfg["headdim"], ngroups=1, mimo_rank=cfg["mimo"])
    H, P, N, M, A = c.nheads, c.per_head_dim, c.state_rank, c.mimo_rank, c.num_rope_angles
    rng = np.random.default_rng(seed)
    L = 1024
    prm = dict(nheads=H, headdim=P, ngroups=1, dstate=N, mimo=M, rope_dim=c.rope_dim,
               dt_bias=np.full(H, -2.0, np.float32), b_norm_w=np.ones(N, np.float32), c_norm_w=np.ones(N, np.float32),
               b_bias=np.ones((H, M, N), np.float32), c_bias=np.ones((H, M, N), np.float32),
               mimo_x=np.full((H, M, P), 1 / M, np.float32))
    proj = rng.standard_normal((1, L, c.d_in_proj)).astype(np.float32)
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    cache = dict(ssm=z(1, H, P, N), k_state=z(1, M, H, N), v_state=z(1, H, P), angle=z(1, H, A))
    t0 = time.perf_counter()
    oracle.mamba3_prep_fwd(proj, prm, cache)
    sec = time.perf_counter() - t0
    total = cfg["batch"] * cfg["seqlen"]
    return {"value": L / sec, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"1 x {L} tokens ({sec:.1f} s) of {total}; float64 numpy restatement of the prologue"}


SSD3_CFG4 = dict(batch=4, seqlen=8192, mimo=4, nheads=32, headdim=64, dstate=128, ngroups=32, chunk=128)


def ssd3_algorithmic(cfg):
    """Compulsory HBM bytes and FLOPs of one Mamba-3 single-SSD call at the
    reference seam (per-head B/C, single_ssd/ssd/serial_recalculated.rs:86-114):
    v, B, C read and y written in bf16, da/gamma/scale f32, final state f32.
    FLOPs (causal-exact, fused L*M axis, per token per head):
    Q M^2 (N + P) + 4 M P N + 2 M^2 (N + P)."""
    b, l, m, h, p, n, q = (cfg[k] for k in ("batch", "seqlen", "mimo", "nheads", "headdim", "dstate", "chunk"))
    tok = b * l
    bytes_ = tok * m * h * (p * 2 * 2 + n * 2 * 2) + tok * h * 3 * 4 + b * h * p * n * 4
    flops = tok * h * (q * m * m * (n + p) + 4 * m * p * n + 2 * m * m * (n + p))
    return bytes_, flops


def make_ssd3_inputs(cfg, dev, seed=0):
    """BASELINE.json configs[4] at the SSD seam: v ~ N(0,1); dt = softplus(N(0,1) + b_h)
    as in config 0; A = -exp(U(ln1, ln16)); da = dt A; lam = sigmoid(N(0,1));
    gamma = lam dt, scale = gamma + (1 - lam_{t+1}) dt_{t+1}; B, C ~ N(0,1)/sqrt(N)
    per head and MIMO rank (the rotation/normalisation upstream of the seam is
    not part of this call)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    b, l, m, h, p, n = (cfg[k] for k in ("batch", "seqlen", "mimo", "nheads", "headdim", "dstate"))
    v = torch.randn((b, l, m, h, p), generator=g, device=dev).to(torch.bfloat16)
    Bm = (torch.randn((b, l, m, h, n), generator=g, device=dev) / n ** 0.5).to(torch.bfloat16)
    Cm = (torch.randn((b, l, m, h, n), generator=g, device=dev) / n ** 0.5).to(torch.bfloat16)
    dt_target = torch.exp(torch.empty(h, device=dev).uniform_(float(torch.log(torch.tensor(1e-3))),
                                                              float(torch.log(torch.tensor(0.1))), generator=g))
    bias = dt_target + torch.log(-torch.expm1(-dt_target))
    dt = torch.nn.functional.softplus(torch.randn((b, l, h), generator=g, device=dev) + bias)
    A = -torch.exp(torch.empty(h, device=dev).uniform_(0.0, float(torch.log(torch.tensor(16.0))), generator=g))
    lam = torch.sigmoid(torch.randn((b, l, h), generator=g, device=dev))
    gamma = lam * dt
    nxt = torch.cat([(1 - lam[:, 1:]) * dt[:, 1:], torch.zeros((b, 1, h), device=dev)], 1)
    return dict(v=v, B=Bm, C=Cm, da=(dt * A).contiguous(), gamma=gamma.contiguous(),
                scale=(gamma + nxt).contiguous())


def bench_ssd3(args):
    import torch

    import mamba_hip
    cfg = dict(SSD3_CFG4)
    dev = torch.device("cuda:0")
    inp = make_ssd3_inputs(cfg, dev)
    y = torch.empty_like(inp["v"])
    hT = torch.empty((cfg["batch"], cfg["nheads"], cfg["headdim"], cfg["dstate"]), device=dev)

    def step(events=None):
        if args.generic:
            _call_events(lambda: mamba_hip.ssd3_fwd(inp["v"], inp["da"], inp["B"], inp["C"], inp["gamma"],
                                                    inp["scale"], None, chunk_len=cfg["chunk"], y=y,
                                                    final_state=hT, generic=True), events)
            return
        mamba_hip.ssd3_fwd(inp["v"], inp["da"], inp["B"], inp["C"], inp["gamma"], inp["scale"], None,
                           chunk_len=cfg["chunk"], y=y, final_state=hT, events=events)

    ms_per_step, kern_ms = _time_steps(args, step)
    nbytes, flops = ssd3_algorithmic(cfg)
    tokens = cfg["batch"] * cfg["seqlen"]
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    tflops = flops / (kern_ms * 1e-3) / 1e12
    # the binding roofline is the one with the longer ideal time
    hbm_bound = nbytes / (HBM_PEAK_GBS * 1e9) >= flops / (BF16_PEAK_TFLOPS * 1e12)
    if hbm_bound:
        roof = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS}
    else:
        roof = {"bound": "mfma", "achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": tflops / BF16_PEAK_TFLOPS}
    roof.update({"traffic": None if args.generic else _profiled_traffic("mamba3_ssd_prefill_cfg4"),
                 "kernel_ms": kern_ms,
                 "algorithmic_bytes": nbytes, "algorithmic_flops": flops, "mfma_tflops": tflops})
    fast = mamba_hip.ssd3_fast_path(inp["v"], inp["da"], inp["B"], inp["C"], inp["gamma"], inp["scale"])
    return {
        "metric": "Mamba-3 SSD prefill tokens/s (B=4 L=8192 H=32 P=64 N=128 MIMO 4) + % HBM roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (BASELINE.json configs[4] distributions at the SSD seam, seed 0)",
        "config": {"workload": "mamba3_ssd_prefill_cfg4" + ("_generic" if args.generic else ""), **cfg,
                   "io": "v/B/C/y bf16 (per-head B/C), da/gamma/scale f32",
                   "entry": "mamba_ssd3_fwd_generic (events around the whole call)" if args.generic
                   else "mamba_ssd3_fwd",
                   "kernel": "generic" if args.generic or not fast else "ssd3_scan_mfma (128 fused positions per chunk)",
                   "hbm_gbs": gbs},
        "roofline": roof,
    }


def mamba3_fused_algorithmic(cfg):
    """Compulsory HBM bytes and the algorithmic FLOPs of the config-4 prefill
    from the in_proj rows to y per rank (mamba3_ssd_fused_fwd): the rows' x,
    raw group-form B / C, dd_dt / dd_A / lambda and rotation columns read once
    (bf16), y per rank written (bf16), the state read and written (f32).
    FLOPs as the SSD seam's (ssd3_algorithmic, chunk 128 steps)."""
    import mamba_hip
    c = mamba_hip.Mamba3Config(d_model=cfg["nheads"] * cfg["headdim"] // 2, state_rank=cfg["dstate"],
                               per_head_dim=cfg["headdim"], ngroups=1, mimo_rank=cfg["mimo"])
    b, L, H, P, N, M, G, A = (cfg["batch"], cfg["seqlen"], c.nheads, c.per_head_dim, c.state_rank, c.mimo_rank,
                              c.ngroups, c.num_rope_angles)
    tok = b * L
    bytes_ = tok * (H * P + 2 * M * G * N + 3 * H + A) * 2 + tok * M * H * P * 2 + 2 * b * H * P * N * 4
    _, flops = ssd3_algorithmic(cfg)
    return bytes_, flops


def bench_mamba3_fused(args):
    """The config-4 Mamba-3 prefill from the in_proj rows to y per rank
    (B=4 L=8192 H=32 P=64 N=128 MIMO 4, full rotation): mamba3_ssd_fused_fwd
    (beta-seed kernel + the fused prologue / SSD scan), reference init.
    ``--mimo`` runs the same head shape at another MIMO rank (1: SISO, the
    reference's default block)."""
    import torch

    import mamba_hip
    cfg = dict(SSD3_CFG4)
    mimo = getattr(args, "mimo", 4)
    cfg["mimo"] = mimo
    wl = "mamba3_fused_prefill_cfg4" if mimo == 4 else f"mamba3_fused_prefill_cfg4_mimo{mimo}"
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    c = mamba_hip.Mamba3Config(d_model=cfg["nheads"] * cfg["headdim"] // 2, state_rank=cfg["dstate"],
                               per_head_dim=cfg["headdim"], ngroups=1, mimo_rank=cfg["mimo"])
    m = c.init(dev, torch.bfloat16, gen)
    b, L = cfg["batch"], cfg["seqlen"]
    proj = torch.randn((b, L, c.d_in_proj), generator=gen, device=dev).to(torch.bfloat16)
    cache = m.new_cache(b)
    a = mamba_hip.mamba3_fused_args(c, proj, cache, dt_bias=m.dt_bias, b_norm_w=m.b_norm_w, c_norm_w=m.c_norm_w,
                                    b_bias=m.b_bias, c_bias=m.c_bias, mimo_x=m.mimo_x, D=m.D)
    if mamba_hip.mamba3_fused_supported(a) != 1:
        raise RuntimeError(f"config 4 at MIMO {mimo} is outside the fused kernel")

    def step(events=None):
        mamba_hip.mamba3_fused_run(a, cache, events)

    ms_per_step, kern_ms = _time_steps(args, step)
    nbytes, flops = mamba3_fused_algorithmic(cfg)
    tokens = b * L
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    tflops = flops / (kern_ms * 1e-3) / 1e12
    hbm_bound = nbytes / (HBM_PEAK_GBS * 1e9) >= flops / (BF16_PEAK_TFLOPS * 1e12)
    if hbm_bound:
        roof = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS}
    else:
        roof = {"bound": "mfma", "achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": tflops / BF16_PEAK_TFLOPS}
    roof.update({"traffic": _profiled_traffic(wl), "kernel_ms": kern_ms,
                 "algorithmic_bytes": nbytes, "algorithmic_flops": flops, "hbm_gbs": gbs,
                 "timing": "HIP events around the seed and fused scan kernels on their stream, per call"})
    return {
        "metric": f"Mamba-3 prefill tokens/s, in_proj rows -> y per rank (B=4 L=8192 H=32 P=64 N=128 MIMO {mimo}) "
                  f"+ % {'MFMA' if not hbm_bound else 'HBM'} roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (config-4 shapes, reference init, in_proj rows ~N(0,1), seed 0)",
        "config": {"workload": wl, **cfg, "rope_dim": c.rope_dim,
                   "io": "proj and y bf16, state f32",
                   "entry": f"mamba3_ssd_fused_fwd (mamba3_seed_kernel + mamba3_ssd_fused<{mimo}>)"},
        "roofline": roof,
    }


def ssd2_bwd_algorithmic(cfg):
    """Causal-exact FLOPs of the Mamba-2 SSD backward at chunk Q = 32, per
    token and head: the reverse chunk loop's four P x N products per position
    (g B_j, g^T x_j, h_c^T dy_j and the state-gradient update) and its five
    lower-triangular Q x Q products (C.B, dy.x, then the dy, C and B
    contractions with them); the chunk-entry states' P x N product.  Bytes: the
    compulsory HBM traffic of the whole call (x, dy, dt, B, C read, f32; dx, ddt,
    dB, dC, d(initial state) written)."""
    b, l, h, p, n, g = (cfg[k] for k in ("batch", "seqlen", "nheads", "headdim", "dstate", "ngroups"))
    q = 32
    th = b * l * h
    chunk_flops = th * 2 * (4 * p * n + (q + 1) / 2 * (3 * n + 2 * p))
    state_flops = th * 2 * p * n
    bytes_ = 4 * (b * l * h * p * 2 + b * l * h + 2 * b * l * g * n) + 4 * (b * l * h * p + b * l * h + 2 * b * l * g * n
                                                                            + b * h * p * n)
    return bytes_, chunk_flops, state_flops


def bench_ssd2_bwd(args):
    """The Mamba-2 SSD backward at the config-1 head shape (B=8 L=4096 H=80
    P=64 N=128, one group), f32: mamba_ssd2_bwd from dy (no initial state, no
    d(final state): a whole-sequence training step)."""
    import torch

    import mamba_hip
    cfg = dict(SSD2_CFG1)
    dev = torch.device("cuda:0")
    inp = make_ssd2_inputs(cfg, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    x, B, C = (inp[k].float() for k in ("x", "B", "C"))
    dy = torch.randn(x.shape, generator=g, device=dev)

    def step(events=None):
        mamba_hip.ssd2_bwd(dy, x, inp["dt"], inp["A"], B, C, inp["D"], None, None, events=events)

    ms_per_step, kern_ms = _time_steps(args, step)
    nbytes, flops, state_flops = ssd2_bwd_algorithmic(cfg)
    tokens = cfg["batch"] * cfg["seqlen"]
    tflops = flops / (kern_ms * 1e-3) / 1e12
    roof = {"bound": "mfma", "achieved": tflops, "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / F32_MFMA_PEAK_TFLOPS, "traffic": _profiled_traffic("mamba2_ssd_bwd_cfg1"),
            "kernel_ms": kern_ms, "algorithmic_flops": flops, "kernel": "ssd2_bwd_chunks (reverse chunk loop)",
            "timing": "HIP events around the reverse chunk-loop kernel on its stream, per call",
            "call_tflops": (flops + state_flops) / (ms_per_step * 1e-3) / 1e12,
            "call_compulsory_bytes": nbytes}
    return {
        "metric": "Mamba-2 SSD backward tokens/s (B=8 L=4096 H=80 P=64 N=128, f32) + % f32 MFMA roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (BASELINE.json configs[1] distributions, dy ~ N(0,1), seeds 0 / 1)",
        "config": {"workload": "mamba2_ssd_bwd_cfg1", **cfg, "chunk": 32, "io": "all f32",
                   "entry": "mamba_ssd2_bwd (chunk states, reverse chunk loop, group sums)"},
        "roofline": roof,
    }


def cpu_baseline_ssd2_bwd(cfg, seed=0):
    """The oracle's float64 token-by-token reverse recurrence (oracle.ssd2_bwd)
    on one sequence of 8192 tokens with every head, scaled to tokens/s."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(seed)
    L, h, p, n = 8192, cfg["nheads"], cfg["headdim"], cfg["dstate"]
    x = rng.standard_normal((1, L, h, p)).astype(np.float32)
    dy = rng.standard_normal((1, L, h, p)).astype(np.float32)
    dt = rng.uniform(1e-3, 0.1, (1, L, h)).astype(np.float32)
    A = -rng.uniform(1.0, 16.0, h).astype(np.float32)
    B = (rng.standard_normal((1, L, 1, n)) / np.sqrt(n)).astype(np.float32)
    C = (rng.standard_normal((1, L, 1, n)) / np.sqrt(n)).astype(np.float32)
    D = rng.standard_normal(h).astype(np.float32)
    t0 = time.perf_counter()
    oracle.ssd2_bwd(dy, None, x, dt, A, B, C, D, None)
    el = time.perf_counter() - t0
    return {"value": L / el, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"1 x {L} tokens, {h} heads ({el:.1f} s), float64 numpy token-by-token reverse "
                      f"recurrence of the reference's backward"}


def ssd3_bwd_algorithmic(cfg):
    """Causal-exact FLOPs of the Mamba-3 single-SSD backward at 32 fused
    positions (32 / M steps) per chunk, per (batch, head): the reverse chunk
    loop's four P x N products per fused position (g B_j, g^T v_j, h_c^T dy_j,
    the state-gradient update) and its five fused Q x Q products (C.B, dy.v,
    then the dy, C and B contractions with them) over the pairs whose step is
    not later, M^2 QS (QS + 1) / 2 per chunk; the chunk-entry states' P x N
    product per fused position."""
    b, l, m, h, p, n = (cfg[k] for k in ("batch", "seqlen", "mimo", "nheads", "headdim", "dstate"))
    qs = 32 // m
    nch = -(-l // qs)
    pairs = m * m * qs * (qs + 1) // 2
    chunk_flops = b * h * nch * 2 * (4 * 32 * p * n + pairs * (3 * n + 2 * p))
    state_flops = b * h * l * m * 2 * p * n
    return chunk_flops, state_flops


def bench_ssd3_bwd(args):
    """The Mamba-3 single-SSD backward at config 4 (B=4 L=8192 H=32 P=64 N=128
    MIMO 4, per-head B / C), f32: mamba_ssd3_bwd from dy (no initial state, no
    d(final state))."""
    import torch

    import mamba_hip
    cfg = dict(SSD3_CFG4)
    dev = torch.device("cuda:0")
    inp = make_ssd3_inputs(cfg, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    v, B, C = (inp[k].float() for k in ("v", "B", "C"))
    dy = torch.randn(v.shape, generator=g, device=dev)

    def step(events=None):
        mamba_hip.ssd3_bwd(dy, v, inp["da"], B, C, inp["gamma"], inp["scale"], None, None, events=events)

    ms_per_step, kern_ms = _time_steps(args, step)
    flops, state_flops = ssd3_bwd_algorithmic(cfg)
    tokens = cfg["batch"] * cfg["seqlen"]
    tflops = flops / (kern_ms * 1e-3) / 1e12
    roof = {"bound": "mfma", "achieved": tflops, "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / F32_MFMA_PEAK_TFLOPS, "traffic": _profiled_traffic("mamba3_ssd_bwd_cfg4"),
            "kernel_ms": kern_ms, "algorithmic_flops": flops, "kernel": "ssd3_bwd_chunks (reverse chunk loop)",
            "timing": "HIP events around the reverse chunk-loop kernel on its stream, per call",
            "call_tflops": (flops + state_flops) / (ms_per_step * 1e-3) / 1e12,
            "grid": f"{cfg['batch'] * cfg['nheads']} workgroups (one per batch row and head) on 256 CUs"}
    return {
        "metric": "Mamba-3 SSD backward tokens/s (B=4 L=8192 H=32 P=64 N=128 MIMO 4, f32) + % f32 MFMA roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (BASELINE.json configs[4] distributions at the SSD seam, dy ~ N(0,1), "
                                "seeds 0 / 1)",
        "config": {"workload": "mamba3_ssd_bwd_cfg4", **cfg, "io": "all f32, per-head B / C",
                   "entry": "mamba_ssd3_bwd (chunk states, reverse chunk loop; 32 fused positions per chunk)"},
        "roofline": roof,
    }


def cpu_baseline_ssd3_bwd(cfg, seed=0):
    """The oracle's float64 token-by-token reverse recurrence (oracle.ssd3_bwd)
    on one sequence of 512 tokens with every head, scaled to tokens/s."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(seed)
    L, m, h, p, n = 512, cfg["mimo"], cfg["nheads"], cfg["headdim"], cfg["dstate"]
    r = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    v, dy = r(1, L, m, h, p), r(1, L, m, h, p)
    B, C = (r(1, L, m, h, n) / np.sqrt(n)).astype(np.float32), (r(1, L, m, h, n) / np.sqrt(n)).astype(np.float32)
    da = (-rng.uniform(1e-3, 0.5, (1, L, h))).astype(np.float32)
    gam = rng.uniform(1e-3, 0.1, (1, L, h)).astype(np.float32)
    scl = rng.uniform(1e-3, 0.2, (1, L, h)).astype(np.float32)
    t0 = time.perf_counter()
    oracle.ssd3_bwd(dy, None, v, da, B, C, gam, scl, None)
    el = time.perf_counter() - t0
    return {"value": L / el, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"1 x {L} tokens, {h} heads, MIMO {m} ({el:.1f} s), float64 numpy token-by-token reverse "
                      f"recurrence of the reference's backward"}


def cpu_baseline_mamba3_fused(cfg, seed=0):
    """oracle.mamba3_prep_fwd then oracle.ssd3 (the f32 C restatement of the
    reference's single-SSD K1-K5) on one sequence of 1024 tokens, scaled to
    tokens/s."""
    import numpy as np

    import mamba_hip
    import oracle
    oracle.build()
    c = mamba_hip.Mamba3Config(d_model=cfg["nheads"] * cfg["headdim"] // 2, state_rank=cfg["dstate"],
                               per_head_dim=cfg["headdim"], ngroups=1, mimo_rank=cfg["mimo"])
    H, P, N, M, A = c.nheads, c.per_head_dim, c.state_rank, c.mimo_rank, c.num_rope_angles
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(seed)
    L = 1024
    prm = dict(nheads=H, headdim=P, ngroups=1, dstate=N, mimo=M, rope_dim=c.rope_dim,
               dt_bias=np.full(H, -2.0, np.float32), b_norm_w=np.ones(N, np.float32), c_norm_w=np.ones(N, np.float32),
               b_bias=np.ones((H, M, N), np.float32), c_bias=np.ones((H, M, N), np.float32),
               mimo_x=np.full((H, M, P), 1 / M, np.float32))
    proj = rng.standard_normal((1, L, c.d_in_proj)).astype(np.float32)
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    cache = dict(ssm=z(1, H, P, N), k_state=z(1, M, H, N), v_state=z(1, H, P), angle=z(1, H, A))
    t0 = time.perf_counter()
    r = oracle.mamba3_prep_fwd(proj, prm, cache)
    oracle.ssd3(r["v"], r["da"], r["B"], r["C"], r["gamma"], r["scale"], r["h0"], chunk=cfg["chunk"], prec=32)
    sec = time.perf_counter() - t0
    total = cfg["batch"] * cfg["seqlen"]
    return {"value": L / sec, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"1 x {L} tokens ({sec:.1f} s) of {total}; float64 numpy prologue + f32 serial single-SSD "
                      f"K1-K5 restatement (OpenMP over heads)"}


def cpu_baseline_ssd3(cfg, seed=0):
    """The f32 CPU restatement of the reference's single-SSD K1-K5 (oracle/,
    OpenMP over (batch, head)) on one sequence of 4096 steps, scaled to tokens/s."""
    import oracle
    from inputs import ssd3_inputs
    oracle.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    L = 4096
    d = ssd3_inputs(seed, 1, L, cfg["mimo"], cfg["nheads"], cfg["headdim"], cfg["dstate"])
    t0 = time.perf_counter()
    oracle.ssd3(d["v"], d["da"], d["B"], d["C"], d["gamma"], d["scale"], None, chunk=cfg["chunk"], prec=32)
    el = time.perf_counter() - t0
    return {"value": L / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"1 x {L} tokens, {cfg['nheads']} heads, MIMO {cfg['mimo']} ({el:.1f} s), f32 serial "
                      f"single-SSD K1-K5 restatement of the reference"}


DECODE_CFG3 = dict(n_layers=64, d_model=2560, expand=2, headdim=64, dstate=128, ngroups=1, conv_kernel=4,
                   batch=64)


def _decode_model_cfg(cfg):
    import mamba_hip
    return mamba_hip.Mamba2Config(d_model=cfg["d_model"], expand=cfg["expand"], per_head_dim=cfg["headdim"],
                                  state_rank=cfg["dstate"], ngroups=cfg["ngroups"],
                                  conv_kernel=cfg["conv_kernel"])


def decode_algorithmic(cfg):
    """Compulsory HBM bytes of one decode step of the stack, and of one launch
    of its state-update kernel.

    Step: every layer's weights read once (in_proj/out_proj bf16, conv weight
    and bias, dt_bias, A, D, both norm gammas f32), every layer's caches read
    and written once (ssm_bhpr and conv_bvk, f32), the token in and the output
    out (f32).  Kernel (one layer): its state tile read and written, its x-channel
    conv windows read and written, the B/C windows read, the in_proj row read
    (bf16), the gated values and per-head sums of squares written (f32)."""
    c = _decode_model_cfg(cfg)
    b, nl = cfg["batch"], cfg["n_layers"]
    H, P, N, K = c.nheads, c.per_head_dim, c.state_rank, c.conv_kernel
    weights = (c.d_model * c.d_in_proj + c.d_inner * c.d_model) * 2 + c.conv_dim * (K + 1) * 4 \
        + 3 * H * 4 + c.d_inner * 4 + c.d_model * 4
    caches = b * (H * P * N + c.conv_dim * K) * 4 * 2
    step_bytes = nl * (weights + caches) + b * c.d_model * 4 * 2
    kernel_bytes = b * (H * P * N * 4 * 2 + c.d_inner * K * 4 * 2 + 2 * c.ngroups * N * K * 4
                        + c.d_in_proj * 2 + c.d_inner * 4 + H * 4)
    return step_bytes, kernel_bytes, weights, caches


def bench_decode(args):
    import torch

    import mamba_hip
    cfg = dict(DECODE_CFG3)
    cfg["batch"] = args.batch
    c = _decode_model_cfg(cfg)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    log(f"init {cfg['n_layers']} layers (bf16 weights, reference init)")
    stack = mamba_hip.Mamba2Stack.init(c, cfg["n_layers"], dev, torch.bfloat16, gen)
    if getattr(args, "no_split", False):
        stack.split_batch = False
    b = cfg["batch"]
    caches = stack.new_caches(b)
    for cc in caches:  # pre-filled states: ssm ~ N(0, 0.1), conv windows ~ N(0, 1)
        cc.ssm_bhpr.normal_(0.0, 0.1, generator=gen)
        cc.conv_bvk.normal_(0.0, 1.0, generator=gen)
    x_in = torch.randn((b, c.d_model), generator=gen, device=dev)
    x_res = torch.empty_like(x_in)
    stack.buffers(b, dev)

    def eager(events=None):
        x_res.copy_(x_in)
        stack.step_(x_res, caches, events)

    log("capture the 64-layer step in a HIP graph")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eager()

    log(f"warmup {args.warmup}")
    warm(graph.replay, args.warmup)
    log(f"timing {args.steps} graph replays")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    # state-update kernel: events around it in every layer of K eager steps
    pairs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(cfg["n_layers"])] for _ in range(args.steps)]
    for ev in pairs:
        eager(ev)
    torch.cuda.synchronize()
    durs = [a.elapsed_time(b_) for ev in pairs for a, b_ in ev]
    kern_ms = sum(durs) / len(durs)
    log(f"ms/step {ms_per_step:.4f}, state-update kernel {kern_ms * 1e3:.2f} us (mean of {len(durs)})")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eager()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step_bytes, kernel_bytes, weights, caches_b = decode_algorithmic(cfg)
    achieved = kernel_bytes / (kern_ms * 1e-3) / 1e9
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    return {
        "metric": f"decode step us at batch {b} (64-layer Mamba-2 2.7B-shaped stack, 1 GPU) + % HBM roofline",
        "value": ms_per_step * 1e3, "unit": "us/step",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (BASELINE.json configs[3]: reference init, states ~N(0,0.1), seed 0)",
        "config": {"workload": "mamba2_decode_step_cfg3", **cfg, "weights": "bf16", "state": "f32",
                   "graph": "hip graph of the whole step", "eager_ms_per_step": eager_ms,
                   "step_bytes": step_bytes, "step_hbm_gbs": step_gbs, "step_hbm_frac": step_gbs / HBM_PEAK_GBS,
                   "entry": ("mamba2_layer_step per layer (packed products, fused norm/residual)" if stack.fused
                             else "mamba_rmsnorm + torch.mm + mamba2_step_ssm + torch.mm per layer"),
                   "schedule": (f"{stack.parts(b)} row parts on {stack.parts(b)} streams" if stack.splits(b)
                                else "one stream")},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel_ms": kern_ms,
                     "algorithmic_bytes": kernel_bytes, "kernel": "step2_ssm_fast<128> (mean over all layers)"},
    }


def cpu_baseline_decode(cfg, budget_s=10.0, seed=0):
    """The f32 CPU restatement of the pre-norm Layer around Mamba2::step
    (oracle/, OpenMP over batch rows) at the same batch, run layer by layer
    until ~budget_s of work, then scaled to the full stack depth."""
    import numpy as np

    import oracle
    oracle.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    c = _decode_model_cfg(cfg)
    b = cfg["batch"]
    rng = np.random.default_rng(seed)
    f = np.float32
    p = dict(pre_norm_w=np.ones(c.d_model, f),
             w_in=rng.uniform(-1, 1, (c.d_model, c.d_in_proj)).astype(f) / np.sqrt(c.d_model).astype(f),
             conv_w=rng.uniform(-0.5, 0.5, (c.conv_dim, c.conv_kernel)).astype(f),
             conv_b=rng.uniform(-0.5, 0.5, c.conv_dim).astype(f),
             dt_bias=np.full(c.nheads, -4.0, f), A=-rng.uniform(1, 16, c.nheads).astype(f),
             D=np.ones(c.nheads, f), norm_w=np.ones(c.d_inner, f),
             w_out=rng.uniform(-1, 1, (c.d_inner, c.d_model)).astype(f) / np.sqrt(c.d_inner).astype(f))
    conv = rng.standard_normal((b, c.conv_dim, c.conv_kernel)).astype(f)
    ssm = (0.1 * rng.standard_normal((b, c.nheads, c.per_head_dim, c.state_rank))).astype(f)
    u = rng.standard_normal((b, c.d_model)).astype(f)
    cd = dict(nheads=c.nheads, headdim=c.per_head_dim, ngroups=c.ngroups, dstate=c.state_rank)
    layers, el = 0, 0.0
    while el < budget_s and layers < cfg["n_layers"]:
        t0 = time.perf_counter()
        u, conv, ssm = oracle.mamba2_layer_step(u, p, conv, ssm, cd, prec=32)
        el += time.perf_counter() - t0
        layers += 1
    us = el / layers * cfg["n_layers"] * 1e6
    return {"value": us, "unit": "us/step", "cores": threads, "kind": "port",
            "sample": f"{layers} of {cfg['n_layers']} layers at batch {b} ({el:.1f} s), scaled to the full "
                      f"stack; f32 restatement of RmsNorm + Mamba2::step + residual"}


COPY_BYTES = 1 << 30


def calibrate_copy():
    """A plain device-to-device copy of COPY_BYTES (read COPY_BYTES, write
    COPY_BYTES): the reference kernel for scaling HBM byte counters."""
    import torch
    src = torch.ones(COPY_BYTES // 4, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 3 x {COPY_BYTES} bytes")


def _profiled_traffic(workload):
    """HBM bytes per launch of the dominant kernel, measured by rocprofv3
    FETCH_SIZE + WRITE_SIZE and scaled by the copy calibration; stored in
    profiles/traffic.json by the profiling run (None when absent)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get(workload)
    return None if entry is None else entry.get("bytes_per_launch")


def _time_steps(args, step):
    """W untimed steps, then K timed back-to-back steps between synchronisations
    (ms/step), then K steps with the library's events around the dominant
    kernel (mean kernel ms)."""
    import torch
    log(f"warmup {args.warmup}")
    warm(step, args.warmup)
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(args.steps)]
    for ev in pairs:
        step(events=ev)
    torch.cuda.synchronize()
    kern_ms = sum(a.elapsed_time(b_) for a, b_ in pairs) / len(pairs)
    log(f"ms/step {ms_per_step:.4f}, dominant kernel {kern_ms:.4f} ms")
    return ms_per_step, kern_ms


def _call_events(call, events):
    """Run call() with torch events recorded around it on the current stream
    (the generic path has no timed entry point: its events bracket the whole
    call, the three SIMT kernels)."""
    if events is not None:
        events[0].record()
    call()
    if events is not None:
        events[1].record()


def bench_ssd2(args):
    import torch

    import mamba_hip
    cfg = dict(SSD2_CFG1)
    dev = torch.device("cuda:0")
    inp = make_ssd2_inputs(cfg, dev)
    b, l, h, p = inp["x"].shape
    y = torch.empty((b, l, h, p), dtype=torch.bfloat16, device=dev)
    hT = torch.empty((b, h, p, cfg["dstate"]), dtype=torch.float32, device=dev)

    def step(events=None):
        if args.generic:
            _call_events(lambda: mamba_hip.ssd2_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"],
                                                    None, chunk_len=cfg["chunk"], y=y, final_state=hT,
                                                    generic=True), events)
            return
        mamba_hip.ssd2_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], None,
                           chunk_len=cfg["chunk"], y=y, final_state=hT, events=events)

    log(f"inputs ready {tuple(inp['x'].shape)}; warmup {args.warmup}")
    warm(step, args.warmup)
    log(f"timing {args.steps} steps")
    # whole-step timing: K back-to-back calls, synchronised on both sides
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_per_step = el * 1e3 / args.steps
    # dominant-kernel timing: HIP events recorded by the library around it
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(args.steps)]
    for ev in pairs:
        step(events=ev)
    torch.cuda.synchronize()
    kern_ms = sum(a.elapsed_time(b_) for a, b_ in pairs) / len(pairs)
    log(f"ms/step {ms_per_step:.3f}, dominant kernel {kern_ms:.3f} ms")
    nbytes, flops = ssd2_algorithmic(cfg)
    tokens = cfg["batch"] * cfg["seqlen"]
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    out = {
        "metric": "SSD prefill tokens/s (Mamba-2 2.7B layer SSD, B=8 L=4096) + % HBM roofline",
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (BASELINE.json configs[1] distributions, seed 0)",
        "config": {"workload": "mamba2_ssd_prefill_cfg1" + ("_generic" if args.generic else ""), **cfg,
                   "io": "x/B/C/y bf16, dt/A/D/state f32",
                   "entry": "mamba_ssd2_fwd_generic (events around the whole call)" if args.generic
                   else "mamba_ssd2_fwd"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel_ms": kern_ms, "algorithmic_bytes": nbytes,
                     "mfma_tflops": flops / (kern_ms * 1e-3) / 1e12,
                     "mfma_frac": flops / (kern_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS},
    }
    return out


MAMBA2_BLOCK_CFG1 = dict(batch=8, seqlen=4096, d_model=2560, chunk=256)


def mamba2_block_algorithmic(cfg):
    """Per-phase compulsory HBM bytes and FLOPs of one Mamba2.forward at the
    config-1 block shape (d_model 2560: 80 heads x 64, d_state 128, one group,
    conv width 4), all activations bf16, states f32:
      in_proj  x read, weight read, zxbcdt written; 2*tok*d_model*d_in_proj flops
      conv     xBC + dt columns read, xbc (bf16) and dt (f32) written, conv window r+w
      ssd      as the SSD workload, plus the initial state read from the cache
      norm     y and z read, normed output written
      out_proj normed output read, weight read, out written; 2*tok*d_inner*d_model flops"""
    import mamba_hip
    c = mamba_hip.Mamba2Config(d_model=cfg["d_model"])
    b, L = cfg["batch"], cfg["seqlen"]
    tok = b * L
    dm, di, dip, cd, H, P, N, K = (c.d_model, c.d_inner, c.d_in_proj, c.conv_dim, c.nheads, c.per_head_dim,
                                   c.state_rank, c.conv_kernel)
    ssd_cfg = dict(batch=b, seqlen=L, nheads=H, headdim=P, dstate=N, ngroups=c.ngroups, chunk=cfg["chunk"])
    ssd_bytes, ssd_flops = ssd2_algorithmic(ssd_cfg)
    return {
        "in_proj": (tok * dm * 2 + dm * dip * 2 + tok * dip * 2, 2 * tok * dm * dip),
        "conv": (tok * (cd + H) * 2 + tok * cd * 2 + tok * H * 4 + 2 * b * cd * K * 4 + cd * (K + 1) * 4 + H * 4,
                 tok * cd * (2 * K + 4)),
        "ssd": (ssd_bytes + b * H * P * N * 4, ssd_flops),
        "norm": (3 * tok * di * 2 + di * 4, 6 * tok * di),
        "out_proj": (tok * di * 2 + di * dm * 2 + tok * dm * 2, 2 * tok * di * dm),
    }


def bench_mamba2_block(args):
    """Mamba2.forward (full block prefill: in_proj -> conv prologue -> SSD ->
    gated RMSNorm -> out_proj) at the config-1 shape, B=8 L=4096, bf16."""
    import torch

    import mamba_hip
    cfg = dict(MAMBA2_BLOCK_CFG1)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    c = mamba_hip.Mamba2Config(d_model=cfg["d_model"])
    m = c.init(dev, torch.bfloat16, gen)
    b, L = cfg["batch"], cfg["seqlen"]
    x = torch.randn((b, L, c.d_model), generator=gen, device=dev).to(torch.bfloat16)
    cache = m.new_cache(b)
    # the SSD inside the block takes the MFMA path on the conv output's views
    xbc = torch.empty((b, L, c.conv_dim), device=dev, dtype=torch.bfloat16)
    di, N = c.d_inner, c.state_rank
    assert mamba_hip.ssd2_fast_path(xbc[:, :, :di].unflatten(2, (c.nheads, c.per_head_dim)),
                                    torch.empty((b, L, c.nheads), device=dev), m.A,
                                    xbc[:, :, di:di + N].unflatten(2, (1, N)),
                                    xbc[:, :, di + N:].unflatten(2, (1, N)), chunk_len=cfg["chunk"])
    del xbc

    def step(events=None):
        m.forward(x, cache, chunk_len=cfg["chunk"], events=events)

    log(f"warmup {args.warmup}")
    warm(step, args.warmup)
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    marks = []
    for _ in range(args.steps):
        ev = []
        step(events=ev)
        marks.append(ev)
    torch.cuda.synchronize()
    names = [n for n, _ in marks[0]][1:]
    phase_ms = {n: sum(ev[i][1].elapsed_time(ev[i + 1][1]) for ev in marks) / len(marks)
                for i, n in enumerate(names)}
    alg = mamba2_block_algorithmic(cfg)
    phases = {}
    for n in names:
        nbytes, flops = alg[n]
        t = phase_ms[n] * 1e-3
        hbm_s, mfma_s = nbytes / (HBM_PEAK_GBS * 1e9), flops / (BF16_PEAK_TFLOPS * 1e12)
        bound = "hbm" if hbm_s >= mfma_s else "mfma"
        achieved = nbytes / t / 1e9 if bound == "hbm" else flops / t / 1e12
        peak = HBM_PEAK_GBS if bound == "hbm" else BF16_PEAK_TFLOPS
        phases[n] = {"ms": phase_ms[n], "bound": bound, "achieved": achieved, "peak": peak,
                     "unit": "GB/s" if bound == "hbm" else "TFLOP/s", "frac": achieved / peak,
                     "algorithmic_bytes": nbytes, "flops": flops}
    log("phases " + ", ".join(f"{n} {phase_ms[n]:.3f} ms ({phases[n]['frac']:.3f})" for n in names))
    dom = max(names, key=lambda n: phase_ms[n])
    d = phases[dom]
    ideal_ms = sum(max(alg[n][0] / (HBM_PEAK_GBS * 1e9), alg[n][1] / (BF16_PEAK_TFLOPS * 1e12)) for n in names) * 1e3
    tokens = b * L
    return {
        "metric": "Mamba-2 block prefill tokens/s (2.7B-shaped layer, B=8 L=4096 d_model 2560) + % roofline",
        "value": tokens / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (reference init of the block, input ~N(0,1), seed 0)",
        "config": {"workload": "mamba2_block_prefill_cfg1", **cfg, "nheads": c.nheads, "headdim": c.per_head_dim,
                   "dstate": c.state_rank, "ngroups": c.ngroups, "conv_kernel": c.conv_kernel,
                   "entry": "Mamba2.forward: torch matmul in_proj/out_proj, mamba2_conv_fwd, mamba_ssd2_fwd, "
                            "mamba2_gated_rmsnorm"},
        "roofline": {"bound": d["bound"], "achieved": d["achieved"], "peak": d["peak"], "unit": d["unit"],
                     "frac": d["frac"], "traffic": None, "kernel": dom, "kernel_ms": d["ms"],
                     "timing": "HIP events on the launch stream between the block's phases, mean over steps",
                     "block_ideal_ms": ideal_ms, "block_frac": ideal_ms / sum(phase_ms.values()),
                     "phases": phases},
    }


def cpu_baseline_mamba2_block(cfg, seed=0):
    """The block on the CPU: in_proj and out_proj as numpy f32 products and
    oracle.mamba2_block_fwd (conv prologue, the f64 serial SSD, gated norm) on
    one batch row of the full length, scaled per token."""
    import numpy as np

    import mamba_hip
    import oracle
    oracle.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    c = mamba_hip.Mamba2Config(d_model=cfg["d_model"])
    rng = np.random.default_rng(seed)
    L = cfg["seqlen"]
    H, P, N, K = c.nheads, c.per_head_dim, c.state_rank, c.conv_kernel
    win = (rng.uniform(-1, 1, (c.d_model, c.d_in_proj)) / np.sqrt(c.d_model)).astype(np.float32)
    wout = (rng.uniform(-1, 1, (c.d_inner, c.d_model)) / np.sqrt(c.d_inner)).astype(np.float32)
    p = dict(conv_w=(rng.uniform(-0.5, 0.5, (c.conv_dim, K))).astype(np.float32),
             conv_b=np.zeros(c.conv_dim, np.float32), dt_bias=np.full(H, -3.0, np.float32),
             A=-np.arange(1, H + 1, dtype=np.float32), D=np.ones(H, np.float32),
             norm_w=np.ones(c.d_inner, np.float32))
    cfgd = dict(nheads=H, headdim=P, ngroups=c.ngroups, dstate=N, norm_before_gate=c.is_norm_before_gate,
                dt_limit=c.dt_limit)
    x = rng.standard_normal((1, L, c.d_model)).astype(np.float32)
    t0 = time.perf_counter()
    proj = x @ win
    yn, _, _ = oracle.mamba2_block_fwd(proj, p, np.zeros((1, c.conv_dim, K), np.float32),
                                       np.zeros((1, H, P, N), np.float32), cfg["chunk"], cfgd)
    _ = yn.astype(np.float32) @ wout
    el = time.perf_counter() - t0
    return {"value": L / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"one batch row of {cfg['batch']} ({L} tokens): numpy f32 in/out products and the "
                      f"oracle's conv, f64 serial SSD and gated norm, {el:.2f} s, per token"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="ssd2",
                    choices=["ssd2", "mamba1", "decode", "ssd3", "mamba3_fused", "mamba1_step", "mamba3_step",
                             "mamba3_prep", "mamba2_block", "ssd2_bwd", "ssd3_bwd", "mamba1_block", "ref_block"])
    ap.add_argument("--ref-mode", default="forward", choices=("forward", "step"),
                    help="ref_block: the reference bench's forward or step group")
    ap.add_argument("--ref-case", default="mamba2",
                    choices=("mamba1", "mamba2", "mamba3/siso", "mamba3/mimo-rank4", "mamba3/siso-double-ssd"),
                    help="ref_block: the reference bench's case")
    ap.add_argument("--mimo", type=int, default=4, choices=(1, 2, 4, 8),
                    help="mamba3_fused: MIMO rank at config 4's head shape (4 is config 4; 1 is SISO)")
    ap.add_argument("--m1-shape", default="ref", choices=sorted(MAMBA1_BLOCK_SHAPES),
                    help="mamba1_block: the reference's bench shape (ref) or config 2's layer shape (cfg2)")
    ap.add_argument("--generic", action="store_true",
                    help="ssd2 / ssd3: run the shape-generic SIMT kernels (the fallback path) instead of the "
                         "MFMA path; the events then bracket the whole call")
    ap.add_argument("--batch", type=int, default=DECODE_CFG3["batch"], help="decode batch")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-split", action="store_true",
                    help="decode / mamba3_step: step the whole batch on one stream (no row-part schedule), "
                         "so that every state-kernel dispatch of a kernel trace covers the full batch")
    ap.add_argument("--m3-stack", action="store_true",
                    help="mamba3_step: step the library's Mamba3Stack (pre-norm residual layers) instead of "
                         "the bare blocks")
    ap.add_argument("--no-decode", action="store_true",
                    help="ssd2 only: leave out the decode_b64 half of the headline metric")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy 3 times (known bytes) so that rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE of the same run can be scaled to true HBM bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the hot path shards by batch/head with no communication)",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "ref_block":
        out = bench_ref_block(args)
        # the reference's own CPU medians of the row are in the line; the oracle
        # baseline of the Mamba-1 block is the one restated at this shape
        base = (lambda: cpu_baseline_mamba1_block("ref")) if args.ref_case == "mamba1" and args.ref_mode == "forward" \
            else None
    elif args.workload == "mamba1_block":
        out = bench_mamba1_block(args)
        base = (lambda: cpu_baseline_mamba1_block(args.m1_shape))
    elif args.workload == "ssd3_bwd":
        out = bench_ssd3_bwd(args)
        base = (lambda: cpu_baseline_ssd3_bwd(SSD3_CFG4))
    elif args.workload == "ssd2_bwd":
        out = bench_ssd2_bwd(args)
        base = (lambda: cpu_baseline_ssd2_bwd(SSD2_CFG1))
    elif args.workload == "mamba2_block":
        out = bench_mamba2_block(args)
        base = (lambda: cpu_baseline_mamba2_block(MAMBA2_BLOCK_CFG1))
    elif args.workload == "mamba3_prep":
        out = bench_mamba3_prep(args)
        base = (lambda: cpu_baseline_mamba3_prep(SSD3_CFG4))
    elif args.workload == "mamba3_step":
        out = bench_mamba3_step(args)
        base = (lambda: cpu_baseline_mamba3_step(MAMBA3_STEP_CFG, args.batch))
    elif args.workload == "mamba1_step":
        out = bench_mamba1_step(args)
        base = (lambda: cpu_baseline_mamba1_step(MAMBA1_STEP_CFG, args.batch))
    elif args.workload == "mamba3_fused":
        out = bench_mamba3_fused(args)
        base = (lambda: cpu_baseline_mamba3_fused(dict(SSD3_CFG4, mimo=args.mimo)))
    elif args.workload == "ssd3":
        out = bench_ssd3(args)
        base = (lambda: cpu_baseline_ssd3(SSD3_CFG4))
    elif args.workload == "decode":
        out = bench_decode(args)
        base = (lambda: cpu_baseline_decode(dict(DECODE_CFG3, batch=args.batch)))
    elif args.workload == "mamba1":
        out = bench_mamba1(args)
        base = (lambda: cpu_baseline_mamba1(MAMBA1_CFG2))
    else:
        out = bench_ssd2(args)
        base = (lambda: cpu_baseline_ssd2(SSD2_CFG1))
    if args.calibrate_copy:
        calibrate_copy()
    traffic = _profiled_traffic(out["config"]["workload"])
    if traffic is not None and out.get("roofline"):
        out["roofline"]["traffic"] = traffic
    if not args.no_cpu_baseline and base is not None:
        log("cpu baseline")
        out["cpu_baseline"] = base()
    if args.workload == "ssd2" and not args.no_decode:
        out["decode_b64"] = decode_b64_summary(args)
    out["warmup_ramp"] = {"min_s": WARMUP_S, "steps_run": _RAMP["steps"], "seconds": round(_RAMP["s"], 3),
                          "note": "untimed steps: the W requested, then more until WARMUP_S s have passed "
                                  "(time-bounded warm-up as the reference's benches/layer.rs)"}
    print(json.dumps(out), flush=True)


def decode_b64_summary(args):
    """The second half of BASELINE.json's headline metric: the recurrent
    decode step of the 64-layer config-3 stack at batch 64 (bench_decode, the
    whole step replayed as one HIP graph, the step methodology of the
    reference's benches/layer.rs:362-395: each step's caches feed the next),
    with the step's HBM fraction, the state-update kernel's roofline and its
    own CPU baseline."""
    import torch
    d = bench_decode(argparse.Namespace(batch=64, steps=args.steps, warmup=args.warmup,
                                        no_split=args.no_split))
    traffic = _profiled_traffic(d["config"]["workload"])
    if traffic is not None:
        d["roofline"]["traffic"] = traffic
    cfg = d["config"]
    s = {"metric": "decode step us at batch 64 (64-layer Mamba-2 2.7B-shaped stack) + % HBM roofline",
         "value": d["value"], "unit": "us/step", "higher_is_better": False, "steps": args.steps,
         "warmup": args.warmup, "step_bytes": cfg["step_bytes"], "step_hbm_gbs": cfg["step_hbm_gbs"],
         "step_hbm_frac": cfg["step_hbm_frac"],
         "target_us": cfg["step_bytes"] / (0.6 * HBM_PEAK_GBS * 1e9) * 1e6,
         "config": {k: cfg[k] for k in ("workload", "batch", "n_layers", "d_model", "nheads", "headdim", "dstate",
                                        "weights", "state", "graph", "eager_ms_per_step", "entry", "schedule")
                    if k in cfg},
         "roofline": d["roofline"]}
    if not args.no_cpu_baseline:
        log("decode cpu baseline")
        s["cpu_baseline"] = cpu_baseline_decode(dict(DECODE_CFG3, batch=64))
    del torch
    return s


if __name__ == "__main__":
    main()
