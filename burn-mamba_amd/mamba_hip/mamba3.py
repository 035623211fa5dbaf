"""Mamba-3 recurrent decode step, mirroring the reference's block signatures.

Reference:
  * ``Mamba3::step(input_bd, Option<cache>) -> (out_bd, cache)``: the double-SSD
    step (src/mamba3/double_ssd/double_ssd/mod.rs:634-760), which single-SSD
    decoding also uses (single_ssd/single_ssd/mod.rs:383-397).
  * ``Mamba3DoubleSsdCache { ssm_bhpr, k_state_bmhr, v_state_bhp, rotation }``
    (double_ssd/cache.rs:81-106) with the Complex2D ``RotationState::Angle``.
  * ``Mamba3Config`` defaults and ``init`` (src/mamba3/mamba3.rs:355-780).

in_proj / out_proj run through ``torch.mm`` (plain library GEMMs); everything
between them is one ``mamba3_step_ssm`` call into libmamba_hip.so.  Nothing
here computes on the CPU; a missing library raises.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import Mamba3FinishArgs, Mamba3FusedArgs, Mamba3PrepArgs, Mamba3StepArgs, check
from .ssd import _dtype_code, _raw_events, _stream
from .step import packed_weight, prefill_mm, prefill_mm_rows, step_mm, step_mm_ok


@dataclass
class Mamba3Cache:
    """ssm_bhpr [b, H, P, N], k_state_bmhr [b, M, H, N] (previous rotated B),
    v_state_bhp [b, H, P] (previous x), angle_bha [b, H, A] (cumulative angle); f32.
    pathway: "single" or "double", the variant of the reference's Mamba3Cache
    (src/mamba3/cache.rs:41-47) that selects the forward pathway; both
    variants hold the same tensors."""
    ssm_bhpr: torch.Tensor
    k_state_bmhr: torch.Tensor
    v_state_bhp: torch.Tensor
    angle_bha: torch.Tensor
    pathway: str = "single"


@dataclass
class Mamba3Config:
    """Mamba3Config (src/mamba3/mamba3.rs:355-470) with the reference defaults
    (Complex2D rotation only)."""
    d_model: int
    state_rank: int = 128
    expand: int = 2
    per_head_dim: int = 64
    ngroups: int = 1
    mimo_rank: int = 1
    a_floor: float = 1e-4
    dt_min: float = 1e-3
    dt_max: float = 0.1
    dt_init_floor: float = 1e-4
    dt_limit: tuple = (0.0, 6.5504e4)
    has_proj_bias: bool = False
    rope_fraction: float = 1.0
    has_outproj_norm: bool = False
    rotation_range: float = 2.0

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def nheads(self) -> int:
        return self.d_inner // self.per_head_dim

    @property
    def rope_dim(self) -> int:
        """rope_dim (mamba3.rs:550-556): state_rank * rope_fraction rounded down to even."""
        d = int(self.state_rank * self.rope_fraction)
        return d - 1 if d % 2 else d

    @property
    def num_rope_angles(self) -> int:
        return max(self.rope_dim // 2, 1)

    @property
    def d_in_proj(self) -> int:
        """d_in_proj (mamba3.rs:600-605)."""
        return (2 * self.d_inner + 2 * self.ngroups * self.state_rank * self.mimo_rank + 3 * self.nheads
                + self.num_rope_angles)

    def init(self, device, dtype=torch.float32, generator: Optional[torch.Generator] = None) -> "Mamba3":
        """Mamba3Config::init (mamba3.rs:632-780): in/out_proj U(+-1/sqrt(fan_in)),
        dt_bias = softplus^-1 of a log-uniform dt, D = 1, norm gammas = 1,
        B/C biases = 1, mimo_x = mimo_o = 1/M, mimo_z = 1."""
        H, M, N, P = self.nheads, self.mimo_rank, self.state_rank, self.per_head_dim

        def uni(shape, bound):
            return (torch.rand(shape, generator=generator, device=device) * 2 - 1) * bound

        in_w = uni((self.d_model, self.d_in_proj), 1 / math.sqrt(self.d_model)).to(dtype)
        out_w = uni((self.d_inner, self.d_model), 1 / math.sqrt(self.d_inner)).to(dtype)
        u = torch.rand(H, generator=generator, device=device)
        dt = torch.exp(u * (math.log(self.dt_max) - math.log(self.dt_min)) + math.log(self.dt_min))
        dt = dt.clamp(min=self.dt_init_floor)
        dt_bias = dt + torch.log(-torch.expm1(-dt))
        ones = lambda *s: torch.ones(s, device=device)  # noqa: E731
        mimo = (M > 1)
        return Mamba3(
            cfg=self, in_proj_w=in_w, out_proj_w=out_w,
            in_proj_b=torch.zeros(self.d_in_proj, device=device) if self.has_proj_bias else None,
            out_proj_b=torch.zeros(self.d_model, device=device) if self.has_proj_bias else None,
            dt_bias=dt_bias.contiguous(), D=ones(H), b_norm_w=ones(N), c_norm_w=ones(N),
            b_bias=ones(H, M, N), c_bias=ones(H, M, N),
            mimo_x=torch.full((H, M, P), 1.0 / M, device=device) if mimo else None,
            mimo_z=ones(H, M, P) if mimo else None,
            mimo_o=torch.full((H, M, P), 1.0 / M, device=device) if mimo else None,
            out_norm_w=ones(P) if self.has_outproj_norm else None)


def _f32c(t, name):
    if t is None:
        return None
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise _lib.MambaHipError(f"{name} must be a contiguous float32 tensor")
    return t


def step_ssm_args(cfg: Mamba3Config, proj: torch.Tensor, cache: Mamba3Cache, *, dt_bias, b_norm_w, c_norm_w,
                  b_bias, c_bias, D=None, mimo_x=None, mimo_z=None, mimo_o=None, out_norm_w=None,
                  out: torch.Tensor) -> Mamba3StepArgs:
    """Fill mamba3_step_args for proj [b, d_in_proj] (f32 or bf16, unit inner stride)."""
    b = proj.shape[0]
    H, P, N, M, G = cfg.nheads, cfg.per_head_dim, cfg.state_rank, cfg.mimo_rank, cfg.ngroups
    A = cfg.num_rope_angles
    if proj.dim() != 2 or proj.shape[1] != cfg.d_in_proj or proj.stride(1) != 1:
        raise _lib.MambaHipError(f"proj must be [b, {cfg.d_in_proj}] with a unit inner stride")
    shapes = dict(ssm_bhpr=(b, H, P, N), k_state_bmhr=(b, M, H, N), v_state_bhp=(b, H, P), angle_bha=(b, H, A))
    for name, shp in shapes.items():
        t = _f32c(getattr(cache, name), name)
        if tuple(t.shape) != shp:
            raise _lib.MambaHipError(f"cache.{name} shape {tuple(t.shape)} != {shp}")
    if out.stride(1) != 1 or tuple(out.shape) != (b, H * P):
        raise _lib.MambaHipError("out must be [b, d_inner] with a unit inner stride")
    a = Mamba3StepArgs()
    a.batch, a.nheads, a.headdim, a.ngroups, a.dstate, a.mimo, a.rope_dim = b, H, P, G, N, M, cfg.rope_dim
    a.proj_dtype, a.out_dtype = _dtype_code(proj), _dtype_code(out)
    a.proj, a.proj_sb = proj.data_ptr(), proj.stride(0)
    a.ssm_state, a.k_state = cache.ssm_bhpr.data_ptr(), cache.k_state_bmhr.data_ptr()
    a.v_state, a.angle = cache.v_state_bhp.data_ptr(), cache.angle_bha.data_ptr()
    a.dt_bias = _f32c(dt_bias, "dt_bias").data_ptr()
    a.a_floor, a.dt_min, a.dt_max = cfg.a_floor, cfg.dt_limit[0], cfg.dt_limit[1]
    a.rotation_range = cfg.rotation_range
    a.b_norm_w, a.c_norm_w = _f32c(b_norm_w, "b_norm_w").data_ptr(), _f32c(c_norm_w, "c_norm_w").data_ptr()
    a.b_bias, a.c_bias = _f32c(b_bias, "b_bias").data_ptr(), _f32c(c_bias, "c_bias").data_ptr()
    for nm, t in (("mimo_x", mimo_x), ("mimo_z", mimo_z), ("mimo_o", mimo_o), ("D", D), ("out_norm_w", out_norm_w)):
        setattr(a, nm, None if t is None else _f32c(t, nm).data_ptr())
    a.out, a.out_sb = out.data_ptr(), out.stride(0)
    return a


def step_ssm(args: Mamba3StepArgs, device, events=None):
    """One mamba3_step_ssm launch on the current stream (events: optional (start, stop))."""
    L = _lib.lib()
    st = _stream(device)
    if events is not None:
        e0, e1 = _raw_events(events, device)
        check(L.mamba3_step_ssm_timed(ctypes.byref(args), st, e0, e1), "mamba3_step_ssm_timed")
    else:
        check(L.mamba3_step_ssm(ctypes.byref(args), st), "mamba3_step_ssm")


def prep_args(cfg: Mamba3Config, proj: torch.Tensor, cache: Mamba3Cache, *, dt_bias, b_norm_w, c_norm_w, b_bias,
              c_bias, mimo_x=None, io_dtype=None, outputs: bool = True) -> Mamba3PrepArgs:
    """The mamba3_prep_args of one call, with its outputs allocated (kept on
    the struct as `outputs` and `angle_out`); outputs=False allocates only the
    initial state (the fused scan's prologue arguments)."""
    b, L, row = proj.shape
    H, P, N, M, G = cfg.nheads, cfg.per_head_dim, cfg.state_rank, cfg.mimo_rank, cfg.ngroups
    if row != cfg.d_in_proj or proj.stride(2) != 1:
        raise _lib.MambaHipError(f"proj must be [b, l, {cfg.d_in_proj}] with a unit inner stride")
    dev, iod = proj.device, io_dtype or proj.dtype
    out = dict(h0=torch.empty((b, H, P, N), device=dev))
    if outputs:
        out.update(v=torch.empty((b, L, M, H, P), device=dev, dtype=iod),
                   B=torch.empty((b, L, M, H, N), device=dev, dtype=iod),
                   C=torch.empty((b, L, M, H, N), device=dev, dtype=iod),
                   da=torch.empty((b, L, H), device=dev), gamma=torch.empty((b, L, H), device=dev),
                   scale=torch.empty((b, L, H), device=dev))
    angle_out = torch.empty_like(cache.angle_bha)
    a = Mamba3PrepArgs()
    a.batch, a.seqlen, a.nheads, a.headdim, a.ngroups, a.dstate, a.mimo = b, L, H, P, G, N, M
    a.rope_dim, a.proj_dtype = cfg.rope_dim, _dtype_code(proj)
    a.io_dtype = _dtype_code(out["v"]) if outputs else _dtype_code(torch.empty(0, dtype=iod))
    a.proj, a.proj_sb, a.proj_sl = proj.data_ptr(), proj.stride(0), proj.stride(1)
    a.ssm_state = _f32c(cache.ssm_bhpr, "ssm_bhpr").data_ptr()
    a.k_state = _f32c(cache.k_state_bmhr, "k_state_bmhr").data_ptr()
    a.v_state = _f32c(cache.v_state_bhp, "v_state_bhp").data_ptr()
    a.angle, a.angle_out = _f32c(cache.angle_bha, "angle_bha").data_ptr(), angle_out.data_ptr()
    a.dt_bias = _f32c(dt_bias, "dt_bias").data_ptr()
    a.a_floor, a.dt_min, a.dt_max, a.rotation_range = cfg.a_floor, cfg.dt_limit[0], cfg.dt_limit[1], cfg.rotation_range
    a.b_norm_w, a.c_norm_w = _f32c(b_norm_w, "b_norm_w").data_ptr(), _f32c(c_norm_w, "c_norm_w").data_ptr()
    a.b_bias, a.c_bias = _f32c(b_bias, "b_bias").data_ptr(), _f32c(c_bias, "c_bias").data_ptr()
    a.mimo_x = None if mimo_x is None else _f32c(mimo_x, "mimo_x").data_ptr()
    if outputs:
        a.v, a.B, a.C = out["v"].data_ptr(), out["B"].data_ptr(), out["C"].data_ptr()
        a.da, a.gamma, a.scale = out["da"].data_ptr(), out["gamma"].data_ptr(), out["scale"].data_ptr()
    a.initial_state = out["h0"].data_ptr()
    a.outputs, a.angle_out_t = out, angle_out
    return a


def prep_fast_path(args: Mamba3PrepArgs) -> int:
    """1 if mamba3_prep_fwd runs the segment-parallel kernels for these
    arguments, 0 for the per-(batch, head, rank) kernel, -1 if invalid."""
    return int(_lib.lib().mamba3_prep_fast_path(ctypes.byref(args)))


def prep_fwd(cfg: Mamba3Config, proj: torch.Tensor, cache: Mamba3Cache, *, dt_bias, b_norm_w, c_norm_w, b_bias,
             c_bias, mimo_x=None, io_dtype=None):
    """mamba3_prep_fwd: proj [b, l, d_in_proj] -> dict(v [b,l,M,H,P], B, C [b,l,M,H,N],
    da, gamma, scale [b,l,H], h0 [b,H,P,N]).  The cache's k_state / v_state are
    replaced in place by the last token's; its angle by the new cumulative angle."""
    a = prep_args(cfg, proj, cache, dt_bias=dt_bias, b_norm_w=b_norm_w, c_norm_w=c_norm_w, b_bias=b_bias,
                  c_bias=c_bias, mimo_x=mimo_x, io_dtype=io_dtype)
    dev = proj.device
    L_ = _lib.lib()
    nws = L_.mamba3_prep_workspace_size(ctypes.byref(a))
    ws = torch.empty(max(int(nws), 1), device=dev, dtype=torch.uint8) if nws else None
    check(L_.mamba3_prep_fwd(ctypes.byref(a), None if ws is None else ws.data_ptr(), int(nws), _stream(dev)),
          "mamba3_prep_fwd")
    cache.angle_bha = a.angle_out_t
    return a.outputs


def fused_args(cfg: Mamba3Config, proj: torch.Tensor, cache: Mamba3Cache, *, dt_bias, b_norm_w, c_norm_w, b_bias,
               c_bias, mimo_x=None, D=None) -> Mamba3FusedArgs:
    """The mamba3_fused_args of one call: the prologue's arguments (without its
    per-head outputs) and y [b, l, M, H, P] bf16 + the final state, allocated
    and kept on the struct as `y_t`, `final_t`, `angle_out_t`."""
    b, L, _ = proj.shape
    H, P, N, M = cfg.nheads, cfg.per_head_dim, cfg.state_rank, cfg.mimo_rank
    pa = prep_args(cfg, proj, cache, dt_bias=dt_bias, b_norm_w=b_norm_w, c_norm_w=c_norm_w, b_bias=b_bias,
                   c_bias=c_bias, mimo_x=mimo_x, io_dtype=torch.bfloat16, outputs=False)
    a = Mamba3FusedArgs()
    a.prep = pa
    y = torch.empty((b, L, M, H, P), device=proj.device, dtype=torch.bfloat16)
    hT = torch.empty((b, H, P, N), device=proj.device)
    a.D = None if D is None else _f32c(D, "D").data_ptr()
    a.y, a.final_state = y.data_ptr(), hT.data_ptr()
    a.y_t, a.final_t, a.angle_out_t, a.h0_t = y, hT, pa.angle_out_t, pa.outputs["h0"]
    return a


def fused_supported(args: Mamba3FusedArgs) -> int:
    """1 if mamba3_ssd_fused_fwd runs for these arguments, 0 if the shape or
    layout is outside the fused kernel, -1 if invalid."""
    return int(_lib.lib().mamba3_ssd_fused_supported(ctypes.byref(args)))


def fused_run(args: Mamba3FusedArgs, cache: Mamba3Cache, events=None):
    """Launch mamba3_ssd_fused_fwd on the current stream; returns (y, final
    state) and points the cache's angle at the new one."""
    dev = args.y_t.device
    L_ = _lib.lib()
    if events is not None:
        e0, e1 = _raw_events(events, dev)
        check(L_.mamba3_ssd_fused_fwd_timed(ctypes.byref(args), _stream(dev), e0, e1), "mamba3_ssd_fused_fwd_timed")
    else:
        check(L_.mamba3_ssd_fused_fwd(ctypes.byref(args), _stream(dev)), "mamba3_ssd_fused_fwd")
    cache.angle_bha = args.angle_out_t
    return args.y_t, args.final_t


def ssd_fused_fwd(cfg: Mamba3Config, proj: torch.Tensor, cache: Mamba3Cache, *, dt_bias, b_norm_w, c_norm_w,
                  b_bias, c_bias, mimo_x=None, D=None, events=None):
    """mamba3_ssd_fused_fwd: proj [b, l, d_in_proj] (bf16) -> (y [b, l, M, H, P]
    bf16 = y_ssd + D v, final state [b, H, P, N] f32), the prologue fused into
    the scan.  The cache's k_state / v_state / angle are replaced as by
    prep_fwd; its ssm_bhpr is read (the caller stores the final state)."""
    a = fused_args(cfg, proj, cache, dt_bias=dt_bias, b_norm_w=b_norm_w, c_norm_w=c_norm_w, b_bias=b_bias,
                   c_bias=c_bias, mimo_x=mimo_x, D=D)
    return fused_run(a, cache, events)


def finish_fwd(cfg: Mamba3Config, y_ssd: torch.Tensor, v: Optional[torch.Tensor], z: torch.Tensor, *, D=None,
               mimo_z=None, mimo_o=None, out_norm_w=None, out: Optional[torch.Tensor] = None):
    """mamba3_finish_fwd: y_ssd [b, l, Y, H, P] whose first M ranks are read (Y = M, or 2M
    for the double pathway's call), v [b, l, M, H, P] (both contiguous; v may be None
    without D, as after the fused scan); z [b, l, H*P] -> [b, l, H*P]."""
    b, L, Y, H, P = y_ssd.shape
    M = cfg.mimo_rank
    if Y < M or (v is not None and tuple(v.shape) != (b, L, M, H, P)):
        raise _lib.MambaHipError("y_ssd must be [b, l, Y >= M, H, P] matching v")
    if v is None and D is not None:
        raise _lib.MambaHipError("v is required with D")
    if not (y_ssd.is_contiguous() and (v is None or (v.is_contiguous() and y_ssd.dtype == v.dtype))) \
            or z.stride(2) != 1:
        raise _lib.MambaHipError("y_ssd / v must be contiguous with one dtype; z needs a unit inner stride")
    if out is None:
        out = torch.empty((b, L, H * P), device=y_ssd.device, dtype=y_ssd.dtype)
    a = Mamba3FinishArgs()
    a.batch, a.seqlen, a.nheads, a.headdim, a.mimo = b, L, H, P, M
    a.y_ranks = Y
    a.io_dtype, a.z_dtype, a.out_dtype = _dtype_code(y_ssd), _dtype_code(z), _dtype_code(out)
    a.y_ssd, a.v = y_ssd.data_ptr(), None if v is None else v.data_ptr()
    a.z, a.z_sb, a.z_sl = z.data_ptr(), z.stride(0), z.stride(1)
    for nm, t in (("D", D), ("mimo_z", mimo_z), ("mimo_o", mimo_o), ("out_norm_w", out_norm_w)):
        setattr(a, nm, None if t is None else _f32c(t, nm).data_ptr())
    a.out, a.out_sb, a.out_sl = out.data_ptr(), out.stride(0), out.stride(1)
    check(_lib.lib().mamba3_finish_fwd(ctypes.byref(a), _stream(y_ssd.device)), "mamba3_finish_fwd")
    return out


def double_inputs(cfg: Mamba3Config, proj: torch.Tensor, prep: dict, x_prev: torch.Tensor, k_prev: torch.Tensor,
                  *, dt_bias, mimo_x=None):
    """mamba3_double_inputs: the 2M-rank inputs (v2, B2, C2) [b, l, 2M, H, P|N] of
    forward_double_ssd's gamma + beta SSD calls, from the prep's v, B, C and the
    cache's x_prev [b, H, P] / K_prev [b, M, H, N] as they were before the prep."""
    v, B, C = prep["v"], prep["B"], prep["C"]
    b, L, M, H, P = v.shape
    N = B.shape[-1]
    if proj.stride(2) != 1 or tuple(proj.shape[:2]) != (b, L):
        raise _lib.MambaHipError("proj must be [b, l, d_in_proj] with a unit inner stride")
    dev = v.device
    v2 = torch.empty((b, L, 2 * M, H, P), device=dev, dtype=v.dtype)
    B2 = torch.empty((b, L, 2 * M, H, N), device=dev, dtype=v.dtype)
    C2 = torch.empty((b, L, 2 * M, H, N), device=dev, dtype=v.dtype)
    a = _lib.Mamba3DoubleInputsArgs()
    a.batch, a.seqlen, a.nheads, a.headdim, a.ngroups, a.dstate, a.mimo = b, L, H, P, cfg.ngroups, N, M
    a.proj_dtype, a.io_dtype = _dtype_code(proj), _dtype_code(v)
    a.proj, a.proj_sb, a.proj_sl = proj.data_ptr(), proj.stride(0), proj.stride(1)
    a.dt_bias = _f32c(dt_bias, "dt_bias").data_ptr()
    a.a_floor, a.dt_min, a.dt_max = cfg.a_floor, cfg.dt_limit[0], cfg.dt_limit[1]
    a.v, a.B, a.C = v.data_ptr(), B.data_ptr(), C.data_ptr()
    a.x_prev, a.k_prev = _f32c(x_prev, "x_prev").data_ptr(), _f32c(k_prev, "k_prev").data_ptr()
    a.mimo_x = None if mimo_x is None else _f32c(mimo_x, "mimo_x").data_ptr()
    a.v2, a.B2, a.C2 = v2.data_ptr(), B2.data_ptr(), C2.data_ptr()
    check(_lib.lib().mamba3_double_inputs(ctypes.byref(a), _stream(dev)), "mamba3_double_inputs")
    return v2, B2, C2


@dataclass
class Mamba3:
    """One Mamba-3 block's parameters (Burn Linear layout [d_in, d_out])."""
    cfg: Mamba3Config
    in_proj_w: torch.Tensor
    out_proj_w: torch.Tensor
    in_proj_b: Optional[torch.Tensor]
    out_proj_b: Optional[torch.Tensor]
    dt_bias: torch.Tensor
    D: torch.Tensor
    b_norm_w: torch.Tensor
    c_norm_w: torch.Tensor
    b_bias: torch.Tensor
    c_bias: torch.Tensor
    mimo_x: Optional[torch.Tensor] = None
    mimo_z: Optional[torch.Tensor] = None
    mimo_o: Optional[torch.Tensor] = None
    out_norm_w: Optional[torch.Tensor] = None

    def new_cache(self, batch: int, pathway: str = "single") -> Mamba3Cache:
        """The reference's fresh cache: zero state, K, v_state and angle
        (double_ssd/double_ssd/mod.rs:649-669); a missing cache is the
        single-ssd variant (mamba3.rs:825-826)."""
        c, dev = self.cfg, self.in_proj_w.device
        z = lambda *s: torch.zeros(s, device=dev)  # noqa: E731
        return Mamba3Cache(z(batch, c.nheads, c.per_head_dim, c.state_rank),
                           z(batch, c.mimo_rank, c.nheads, c.state_rank),
                           z(batch, c.nheads, c.per_head_dim), z(batch, c.nheads, c.num_rope_angles), pathway)

    def _in_proj(self, x: torch.Tensor):
        """in_proj into rows padded to 8 elements (a strided [b, l, d_in_proj]
        view), the layout the prologue's fast kernels read."""
        b, L, _ = x.shape
        wdt = self.in_proj_w.dtype
        proj = prefill_mm_rows(x.reshape(b * L, -1).to(wdt), self.in_proj_w).reshape(b, L, -1)
        if self.in_proj_b is not None:
            proj.add_(self.in_proj_b.to(wdt))
        return proj

    def _out_proj(self, y: torch.Tensor, x: torch.Tensor):
        b, L, _ = y.shape
        out = prefill_mm(y.reshape(b * L, -1), self.out_proj_w).reshape(b, L, -1)
        if self.out_proj_b is not None:
            out = out + self.out_proj_b.to(self.in_proj_w.dtype)
        return out.to(x.dtype)

    def forward(self, x: torch.Tensor, cache: Optional[Mamba3Cache] = None, chunk_len: int = 64):
        """Mamba3::forward (mamba3.rs:805-840): x [b, l, d_model] -> (out [b, l, d_model],
        cache), the pathway chosen by the cache's variant (a missing cache is the
        single-ssd one).  Both pathways compute the same function."""
        if cache is not None and cache.pathway == "double":
            return self.forward_double_ssd(x, cache, chunk_len)
        return self.forward_single_ssd(x, cache, chunk_len)

    def forward_single_ssd(self, x: torch.Tensor, cache: Optional[Mamba3Cache] = None, chunk_len: int = 64):
        """Mamba3::forward_single_ssd (single_ssd/single_ssd/mod.rs:44-360): in_proj /
        out_proj on torch.mm; in between, the fused prologue + scan
        (mamba3_ssd_fused_fwd) where its shape applies, else prep ->
        mamba_ssd3_fwd; then finish."""
        from .ssd3 import ssd3_fwd
        if cache is None:
            cache = self.new_cache(x.shape[0])
        proj = self._in_proj(x)
        if proj.dtype == torch.bfloat16:
            fa = fused_args(self.cfg, proj, cache, dt_bias=self.dt_bias, b_norm_w=self.b_norm_w,
                            c_norm_w=self.c_norm_w, b_bias=self.b_bias, c_bias=self.c_bias, mimo_x=self.mimo_x,
                            D=self.D)
            if fused_supported(fa) == 1:
                y_ssd, hT = fused_run(fa, cache)
                cache.ssm_bhpr = hT
                y = finish_fwd(self.cfg, y_ssd, None, proj[:, :, :self.cfg.d_inner], mimo_z=self.mimo_z,
                               mimo_o=self.mimo_o, out_norm_w=self.out_norm_w)
                return self._out_proj(y, x), cache
        pr = prep_fwd(self.cfg, proj, cache, dt_bias=self.dt_bias, b_norm_w=self.b_norm_w, c_norm_w=self.c_norm_w,
                      b_bias=self.b_bias, c_bias=self.c_bias, mimo_x=self.mimo_x)
        y_ssd, hT = ssd3_fwd(pr["v"], pr["da"], pr["B"], pr["C"], pr["gamma"], pr["scale"], pr["h0"],
                             chunk_len=chunk_len)
        cache.ssm_bhpr = hT
        y = finish_fwd(self.cfg, y_ssd, pr["v"], proj[:, :, :self.cfg.d_inner], D=self.D, mimo_z=self.mimo_z,
                       mimo_o=self.mimo_o, out_norm_w=self.out_norm_w)
        return self._out_proj(y, x), cache

    def forward_double_ssd(self, x: torch.Tensor, cache: Optional[Mamba3Cache] = None, chunk_len: int = 64):
        """Mamba3::forward_double_ssd (double_ssd/double_ssd/mod.rs:40-369): the same
        prep (QK-norm, bias, rotation, coefficients), then the gamma and beta SSD
        calls of :254-283 as one 2M-rank mamba_ssd3_double_fwd (they share da and
        C, so the first M ranks of its y are y_gamma + y_beta and its final state
        is their sum), then the D skip / gate / merge and out_proj."""
        from .ssd3 import ssd3_double_fwd
        if cache is None:
            cache = self.new_cache(x.shape[0], "double")
        proj = self._in_proj(x)
        # the beta term's t = 0 inputs: x_prev and K_prev before the prep replaces them
        x_prev, k_prev = cache.v_state_bhp.clone(), cache.k_state_bmhr.clone()
        pr = prep_fwd(self.cfg, proj, cache, dt_bias=self.dt_bias, b_norm_w=self.b_norm_w, c_norm_w=self.c_norm_w,
                      b_bias=self.b_bias, c_bias=self.c_bias, mimo_x=self.mimo_x)
        v2, B2, C2 = double_inputs(self.cfg, proj, pr, x_prev, k_prev, dt_bias=self.dt_bias, mimo_x=self.mimo_x)
        y2, hT = ssd3_double_fwd(v2, pr["da"], B2, C2, cache.ssm_bhpr, chunk_len=chunk_len)
        cache.ssm_bhpr = hT
        y = finish_fwd(self.cfg, y2, pr["v"], proj[:, :, :self.cfg.d_inner], D=self.D, mimo_z=self.mimo_z,
                       mimo_o=self.mimo_o, out_norm_w=self.out_norm_w)
        return self._out_proj(y, x), cache

    def step(self, x: torch.Tensor, cache: Optional[Mamba3Cache] = None, events=None):
        """Mamba3::step: x [b, d_model] -> (out [b, d_model], cache updated in place)."""
        if cache is None:
            cache = self.new_cache(x.shape[0])
        wdt = self.in_proj_w.dtype
        xw = x.to(wdt)
        b = x.shape[0]
        # the packed streaming product where it applies (bf16 weights, d_in a
        # multiple of 16, at most 256 rows); its outputs are rounded to the
        # weight dtype, as the library GEMM's are
        if step_mm_ok(xw, self.in_proj_w):
            proj = step_mm(xw, self.in_proj_w, out=torch.empty((b, self.cfg.d_in_proj), dtype=wdt, device=x.device))
        else:
            proj = torch.mm(xw, self.in_proj_w)
        if self.in_proj_b is not None:
            proj = proj + self.in_proj_b.to(proj.dtype)
        y = torch.empty((b, self.cfg.d_inner), dtype=wdt, device=x.device)
        args = step_ssm_args(self.cfg, proj, cache, dt_bias=self.dt_bias, b_norm_w=self.b_norm_w,
                             c_norm_w=self.c_norm_w, b_bias=self.b_bias, c_bias=self.c_bias, D=self.D,
                             mimo_x=self.mimo_x, mimo_z=self.mimo_z, mimo_o=self.mimo_o,
                             out_norm_w=self.out_norm_w, out=y)
        step_ssm(args, x.device, events)
        if step_mm_ok(y, self.out_proj_w):
            out = step_mm(y, self.out_proj_w, out=torch.empty((b, self.cfg.d_model), dtype=wdt, device=x.device))
        else:
            out = torch.mm(y, self.out_proj_w)
        if self.out_proj_b is not None:
            out = out + self.out_proj_b.to(out.dtype)
        return out.to(x.dtype), cache

    def pack_products(self) -> None:
        """Make the packed copies of in_proj / out_proj that step() streams
        (bf16 weights only), so that no packing happens inside a captured HIP
        graph.  step() packs on first use otherwise."""
        for w in (self.in_proj_w, self.out_proj_w):
            if w.dtype == torch.bfloat16 and w.shape[0] % 16 == 0:
                packed_weight(w)


@dataclass
class Mamba3Layer:
    """Pre-norm residual layer (src/modules/layer.rs:224-232) around a Mamba3 block."""
    norm_w: torch.Tensor   # [d_model] f32 RmsNorm gamma
    mixer: Mamba3


class Mamba3Stack:
    """A stack of pre-norm Mamba3 layers stepped one token at a time
    (Layers::step, src/modules/layers.rs:427-520, without class latents; each
    layer Layer::step_one, layer.rs:224-232).

    The residual stream is kept in f32.  Per layer: one mamba_rmsnorm (the
    previous layer's residual add fused with this layer's pre-norm, into a bf16
    operand), in_proj on the packed streaming product, mamba3_step_ssm,
    out_proj; a last mamba_rmsnorm adds the final residual.  bf16 blocks whose
    products the packed kernel takes (d_model and d_inner multiples of 16).
    Buffers and step arguments are made once per batch size, so ``step_``
    allocates nothing and can be captured in a HIP graph.  With
    ``split_batch`` (the default) a batch of 34 to 256 rows steps as row
    parts of at most 32 rows on up to four streams (``batch_parts``): one
    part's weight-streaming products overlap another part's step kernel
    (each part reads the weights once; rows never interact).  Mamba-3's
    weights are small next to its caches, so more parts pay here where they
    do not for Mamba2Stack: at 96 / 100 / 256 rows three or four parts
    measured 4.31 -> 4.01, 4.49 -> 4.19 and 9.41 -> 8.61 ms per 64-block step
    against two (eight at 256 rows: 10.07 ms)."""

    max_parts = 4

    def __init__(self, layers, split_batch: bool = True):
        from .step import linear  # noqa: F401  (fails early if the product entry is missing)
        assert layers
        self.layers = list(layers)
        self.cfg = self.layers[0].mixer.cfg
        c = self.cfg
        for l in self.layers:
            m = l.mixer
            if m.in_proj_w.dtype != torch.bfloat16 or m.out_proj_w.dtype != torch.bfloat16:
                raise _lib.MambaHipError("Mamba3Stack steps bf16 blocks (packed products)")
        if c.d_model % 16 or c.d_inner % 16:
            raise _lib.MambaHipError("Mamba3Stack needs d_model and d_inner multiples of 16")
        self.split_batch = split_batch
        self._packed = [(packed_weight(l.mixer.in_proj_w), packed_weight(l.mixer.out_proj_w)) for l in self.layers]
        self._bias = [tuple(None if t is None else t.float().contiguous()
                            for t in (l.mixer.in_proj_b, l.mixer.out_proj_b)) for l in self.layers]
        self._bufs = {}
        self._args = {}
        self._side = None

    @staticmethod
    def init(cfg: Mamba3Config, n_layers: int, device, dtype=torch.bfloat16,
             generator: Optional[torch.Generator] = None, split_batch: bool = True) -> "Mamba3Stack":
        return Mamba3Stack([Mamba3Layer(norm_w=torch.ones(cfg.d_model, device=device, dtype=torch.float32),
                                        mixer=cfg.init(device, dtype, generator)) for _ in range(n_layers)],
                           split_batch=split_batch)

    def new_caches(self, batch: int, pathway: str = "single"):
        return [l.mixer.new_cache(batch, pathway) for l in self.layers]

    def parts(self, b: int) -> int:
        """Row parts of an untimed step of batch ``b``, each on its own stream (batch_parts)."""
        from .step import batch_parts
        return batch_parts(b, self.max_parts) if self.split_batch else 1

    def splits(self, b: int) -> bool:
        """Whether an untimed step of batch ``b`` runs as row parts on several streams."""
        return self.parts(b) > 1

    def buffers(self, batch: int, device, slot: int = 0):
        key = (batch, str(device), slot)
        if key not in self._bufs:
            from ._lib import LinearArgs
            c = self.cfg
            bf = torch.bfloat16
            bufs = dict(
                normed=torch.empty((batch, c.d_model), device=device, dtype=bf),
                proj=torch.empty((batch, c.d_in_proj), device=device, dtype=bf),
                y=torch.empty((batch, c.d_inner), device=device, dtype=bf),
                out=torch.empty((batch, c.d_model), device=device, dtype=bf))
            # one workspace for both products (used in order): the larger need
            need = 256
            for d_in, d_out in ((c.d_model, c.d_in_proj), (c.d_inner, c.d_model)):
                la = LinearArgs()
                la.rows, la.d_in, la.d_out = batch, d_in, d_out
                la.x_dtype = la.y_dtype = _lib.MAMBA_BF16
                la.x_ld, la.y_ld = d_in, d_out
                need = max(need, _lib.lib().mamba_linear_workspace_size(ctypes.byref(la)))
            bufs["ws"] = torch.empty(need, device=device, dtype=torch.uint8)
            self._bufs[key] = bufs
        return self._bufs[key]

    def _layer_args(self, i: int, slot: int, bufs, cache: Mamba3Cache) -> Mamba3StepArgs:
        key = (i, slot, bufs["proj"].data_ptr(), cache.ssm_bhpr.data_ptr(), cache.k_state_bmhr.data_ptr(),
               cache.v_state_bhp.data_ptr(), cache.angle_bha.data_ptr(), cache.ssm_bhpr.shape[0])
        a = self._args.get(key)
        if a is None:
            m = self.layers[i].mixer
            a = step_ssm_args(self.cfg, bufs["proj"], cache, dt_bias=m.dt_bias, b_norm_w=m.b_norm_w,
                              c_norm_w=m.c_norm_w, b_bias=m.b_bias, c_bias=m.c_bias, D=m.D, mimo_x=m.mimo_x,
                              mimo_z=m.mimo_z, mimo_o=m.mimo_o, out_norm_w=m.out_norm_w, out=bufs["y"])
            self._args[key] = a
        return a

    def _run(self, x_res: torch.Tensor, caches, events, slot: int):
        from .step import linear, rmsnorm
        c = self.cfg
        bufs = self.buffers(x_res.shape[0], x_res.device, slot)
        prev = None
        for i, layer in enumerate(self.layers):
            rmsnorm(x_res, layer.norm_w, out=bufs["normed"], add=prev)
            (pin, pout), (bin_, bout) = self._packed[i], self._bias[i]
            linear(bufs["normed"], pin, c.d_in_proj, bias=bin_, out=bufs["proj"], workspace=bufs["ws"])
            step_ssm(self._layer_args(i, slot, bufs, caches[i]), x_res.device, None if events is None else events[i])
            linear(bufs["y"], pout, c.d_model, bias=bout, out=bufs["out"], workspace=bufs["ws"])
            prev = bufs["out"]
        rmsnorm(x_res, None, add=prev)
        return x_res

    def step_(self, x_res: torch.Tensor, caches, events=None):
        """In-place step of the whole stack: x_res [b, d_model] f32 becomes the
        stack output.  ``events``: optional list of one torch.cuda.Event pair per
        layer, recorded around that layer's mamba3_step_ssm (one stream)."""
        if x_res.dtype != torch.float32 or x_res.dim() != 2 or x_res.stride(1) != 1:
            raise _lib.MambaHipError("x_res must be a row-contiguous [b, d_model] float32 tensor")
        b = x_res.shape[0]
        K = self.parts(b) if events is None else 1
        if K > 1:
            cur = torch.cuda.current_stream(x_res.device)
            if self._side is None or len(self._side) < K:
                self._side = tuple(torch.cuda.Stream(x_res.device) for _ in range(K))
            bounds = [(b * k) // K for k in range(K + 1)]
            for k in range(K):
                lo, hi = bounds[k], bounds[k + 1]
                st = self._side[k]
                st.wait_stream(cur)
                with torch.cuda.stream(st):
                    part = [Mamba3Cache(cc.ssm_bhpr[lo:hi], cc.k_state_bmhr[lo:hi], cc.v_state_bhp[lo:hi],
                                        cc.angle_bha[lo:hi], cc.pathway) for cc in caches]
                    self._run(x_res[lo:hi], part, None, 1 + k)
            for st in self._side[:K]:
                cur.wait_stream(st)
            return x_res
        return self._run(x_res, caches, events, 0)

    def step(self, x: torch.Tensor, caches=None):
        """Out-of-place convenience: returns (y [b, d_model] f32, caches)."""
        if caches is None:
            caches = self.new_caches(x.shape[0])
        x_res = x.to(torch.float32).clone()
        self.step_(x_res, caches)
        return x_res, caches
