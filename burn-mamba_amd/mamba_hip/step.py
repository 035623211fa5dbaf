"""Mamba-2 recurrent decode step, mirroring the reference's block signatures.

Reference:
  * ``Mamba2::step(input_bm, Option<Mamba2Cache>) -> (out_bm, Mamba2Cache)``
    (src/mamba2/mamba2.rs:820-1004)
  * ``Mamba2Cache { conv_bvk, ssm_bhpr }`` (src/mamba2/cache.rs:98-122)
  * ``Mamba2Config`` defaults and ``init`` (src/mamba2/mamba2.rs:250-505)
  * the pre-norm ``Layer::step_one`` (src/modules/layer.rs:224-232):
    ``x + block_step(RmsNorm(x))``.

The in_proj / out_proj products run on the ROCm BLAS through ``torch.mm``
(plain library GEMMs); everything between them (conv window, softplus, state
update, readout, gated RMSNorm) is one ``mamba2_step_ssm`` call into
libmamba_hip.so, and the residual + pre-norm is one ``mamba_rmsnorm`` call.
Nothing here computes on the CPU; a missing library raises.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import torch

from . import _lib
from ._lib import LinearArgs, Mamba2LayerArgs, Mamba2StepArgs, RmsNormArgs, check
from .ssd import _dtype_code, _raw_events, _stream


@dataclass
class Mamba2Cache:
    """conv_bvk [batch, conv_dim, conv_kernel] and ssm_bhpr [batch, nheads, headdim, dstate], f32."""
    conv_bvk: torch.Tensor
    ssm_bhpr: torch.Tensor


@dataclass
class Mamba2Config:
    """Mamba2Config (src/mamba2/mamba2.rs:250-330) with the reference defaults."""
    d_model: int
    state_rank: int = 128
    conv_kernel: int = 4
    expand: int = 2
    per_head_dim: int = 64
    ngroups: int = 1
    a_init_range: Tuple[float, float] = (1.0, 16.0)
    is_norm_before_gate: bool = False
    dt_min: float = 1e-3
    dt_max: float = 0.1
    dt_init_floor: float = 1e-4
    dt_limit: Tuple[float, float] = (0.0, 6.5504e4)
    has_proj_bias: bool = False
    has_conv_bias: bool = True

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def nheads(self) -> int:
        return self.d_inner // self.per_head_dim

    @property
    def conv_dim(self) -> int:
        return self.d_inner + 2 * self.ngroups * self.state_rank

    @property
    def d_in_proj(self) -> int:
        return self.d_inner + self.conv_dim + self.nheads

    def init(self, device, dtype=torch.bfloat16, generator: Optional[torch.Generator] = None) -> "Mamba2":
        """Random init following Mamba2Config::init (mamba2.rs:391-505).

        Projection weights are stored in ``dtype`` ([d_in, d_out], Burn's Linear
        layout); the per-channel parameters stay f32.  Values are drawn on the
        generator's device (CPU when no generator is given)."""
        assert self.nheads * self.per_head_dim == self.d_inner and self.nheads % self.ngroups == 0
        g = generator
        gdev = g.device if g is not None else torch.device("cpu")

        def rand(shape):
            return torch.rand(shape, generator=g, device=gdev, dtype=torch.float32)

        def uni(shape, fan_in):
            bound = 1.0 / math.sqrt(fan_in)
            return (rand(shape) * 2 - 1) * bound

        H = self.nheads
        in_w = uni((self.d_model, self.d_in_proj), self.d_model)
        conv_w = uni((self.conv_dim, self.conv_kernel), self.conv_kernel)
        conv_b = uni((self.conv_dim,), self.conv_kernel) if self.has_conv_bias else None
        lo, hi = math.log(self.dt_min), math.log(self.dt_max)
        dt = torch.exp(rand(H).double() * (hi - lo) + lo)
        dt = dt.clamp(min=self.dt_init_floor)
        dt_bias = dt + torch.log(-torch.expm1(-dt))
        a0, a1 = self.a_init_range
        a_log = torch.log(rand(H).double() * (a1 - a0) + a0)
        out_w = uni((self.d_inner, self.d_model), self.d_inner)
        f32 = dict(device=device, dtype=torch.float32)
        return Mamba2(
            cfg=self,
            in_proj_w=in_w.to(device=device, dtype=dtype),
            in_proj_b=torch.zeros(self.d_in_proj, device=device, dtype=dtype) if self.has_proj_bias else None,
            conv_w=conv_w.to(**f32),
            conv_b=None if conv_b is None else conv_b.to(**f32),
            dt_bias=dt_bias.to(**f32),
            a_log=a_log.to(**f32),
            d=torch.ones(H, **f32),
            norm_w=torch.ones(self.d_inner, **f32),
            out_proj_w=out_w.to(device=device, dtype=dtype),
            out_proj_b=torch.zeros(self.d_model, device=device, dtype=dtype) if self.has_proj_bias else None,
        )


def step_ssm_args(cfg: Mamba2Config, zxbcdt: torch.Tensor, cache: Mamba2Cache, conv_w, conv_b, dt_bias,
                  A, D, norm_w, out: torch.Tensor) -> Mamba2StepArgs:
    b = zxbcdt.shape[0]
    if zxbcdt.stride(-1) != 1 or out.stride(-1) != 1:
        raise _lib.MambaHipError("zxbcdt and out need a contiguous last axis")
    for t, nm in ((cache.conv_bvk, "conv_bvk"), (cache.ssm_bhpr, "ssm_bhpr"), (conv_w, "conv_w")):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise _lib.MambaHipError(f"{nm} must be contiguous float32")
    if tuple(cache.ssm_bhpr.shape) != (b, cfg.nheads, cfg.per_head_dim, cfg.state_rank):
        raise _lib.MambaHipError(f"ssm_bhpr shape {tuple(cache.ssm_bhpr.shape)} does not match the config")
    if tuple(cache.conv_bvk.shape) != (b, cfg.conv_dim, cfg.conv_kernel):
        raise _lib.MambaHipError(f"conv_bvk shape {tuple(cache.conv_bvk.shape)} does not match the config")
    if zxbcdt.shape[1] != cfg.d_in_proj or out.shape != (b, cfg.d_inner):
        raise _lib.MambaHipError("zxbcdt / out shapes do not match the config")
    a = Mamba2StepArgs()
    a.batch, a.nheads, a.headdim = b, cfg.nheads, cfg.per_head_dim
    a.ngroups, a.dstate, a.conv_kernel = cfg.ngroups, cfg.state_rank, cfg.conv_kernel
    a.zxbcdt_dtype, a.out_dtype = _dtype_code(zxbcdt), _dtype_code(out)
    a.norm_before_gate = int(cfg.is_norm_before_gate)
    a.zxbcdt, a.zxbcdt_sb = zxbcdt.data_ptr(), zxbcdt.stride(0)
    a.conv_state, a.conv_w = cache.conv_bvk.data_ptr(), conv_w.data_ptr()
    a.conv_b = None if conv_b is None else conv_b.data_ptr()
    a.dt_bias = None if dt_bias is None else dt_bias.data_ptr()
    a.A = A.data_ptr()
    a.D = None if D is None else D.data_ptr()
    a.dt_min, a.dt_max = float(cfg.dt_limit[0]), float(cfg.dt_limit[1])
    a.norm_w, a.ssm_state = norm_w.data_ptr(), cache.ssm_bhpr.data_ptr()
    a.out, a.out_sb = out.data_ptr(), out.stride(0)
    return a


def step_ssm(args: Mamba2StepArgs, workspace: torch.Tensor, events=None):
    """One mamba2_step_ssm call on the current stream (workspace: uint8 device buffer).

    ``events``: optional torch.cuda.Event pair recorded around the state-update kernel."""
    L = _lib.lib()
    need = L.mamba2_step_workspace_size(ctypes.byref(args))
    if workspace.numel() < need:
        raise _lib.MambaHipError(f"workspace of {need} bytes required, got {workspace.numel()}")
    stream = _stream(workspace.device)
    if events is None:
        check(L.mamba2_step_ssm(ctypes.byref(args), ctypes.c_void_p(workspace.data_ptr()), need, stream),
              "mamba2_step_ssm")
    else:
        e0, e1 = _raw_events(events, workspace.device)
        check(L.mamba2_step_ssm_timed(ctypes.byref(args), ctypes.c_void_p(workspace.data_ptr()), need, stream,
                                      e0, e1),
              "mamba2_step_ssm_timed")


def rmsnorm(x: torch.Tensor, weight: Optional[torch.Tensor], out: Optional[torch.Tensor] = None,
            add: Optional[torch.Tensor] = None):
    """x += add (when given, in place); out = RmsNorm(x) * weight (when out is given)."""
    if x.dtype != torch.float32 or x.dim() != 2 or x.stride(1) != 1:
        raise _lib.MambaHipError("x must be a row-contiguous 2-d float32 tensor")
    a = RmsNormArgs()
    a.rows, a.cols = x.shape
    a.x, a.x_sr = x.data_ptr(), x.stride(0)
    a.add_dtype = a.out_dtype = 0
    if add is not None:
        if add.shape != x.shape or add.stride(1) != 1:
            raise _lib.MambaHipError("add must match x")
        a.add, a.add_sr, a.add_dtype = add.data_ptr(), add.stride(0), _dtype_code(add)
    if out is not None:
        if out.shape != x.shape or out.stride(1) != 1 or weight is None:
            raise _lib.MambaHipError("out must match x and needs weight")
        a.out, a.out_sr, a.out_dtype = out.data_ptr(), out.stride(0), _dtype_code(out)
        a.weight = weight.data_ptr()
    check(_lib.lib().mamba_rmsnorm(ctypes.byref(a), _stream(x.device)), "mamba_rmsnorm")


def pack_linear(weight: torch.Tensor) -> torch.Tensor:
    """Pack a Linear weight [d_in, d_out] (f32/bf16) for mamba_linear_fwd and the
    fused layer step (done once, at model load).  Returns a uint8 device buffer."""
    d_in, d_out = weight.shape
    if weight.stride(1) != 1:
        raise _lib.MambaHipError("weight needs a contiguous d_out axis")
    L = _lib.lib()
    n = L.mamba_linear_packed_size(d_in, d_out)
    if n == 0:
        raise _lib.MambaHipError(f"unsupported Linear shape {d_in} x {d_out} (d_in must be a multiple of 16)")
    out = torch.empty(n, dtype=torch.uint8, device=weight.device)
    check(L.mamba_linear_pack(ctypes.c_void_p(weight.data_ptr()), d_in, d_out, weight.stride(0),
                              _dtype_code(weight), ctypes.c_void_p(out.data_ptr()), _stream(weight.device)),
          "mamba_linear_pack")
    return out


def linear(x: torch.Tensor, packed_w: torch.Tensor, d_out: int, bias: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x W (+bias) through mamba_linear_fwd (rows <= 256, W packed by pack_linear)."""
    if x.dim() != 2 or x.stride(1) != 1:
        raise _lib.MambaHipError("x must be 2-d with a contiguous last axis")
    rows, d_in = x.shape
    if out is None:
        out = torch.empty(rows, d_out, dtype=torch.float32, device=x.device)
    a = LinearArgs()
    a.rows, a.d_in, a.d_out = rows, d_in, d_out
    a.x_dtype, a.y_dtype = _dtype_code(x), _dtype_code(out)
    a.x, a.x_ld = x.data_ptr(), x.stride(0)
    a.packed_w = packed_w.data_ptr()
    a.bias = None if bias is None else bias.data_ptr()
    a.y, a.y_ld = out.data_ptr(), out.stride(0)
    L = _lib.lib()
    need = L.mamba_linear_workspace_size(ctypes.byref(a))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    check(L.mamba_linear_fwd(ctypes.byref(a), ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
                             _stream(x.device)), "mamba_linear_fwd")
    return out


# every derived copy is kept on the weight under an attribute with this prefix
_DERIVED_PREFIX = "_mamba_"


def _weight_key(w: torch.Tensor):
    """What identifies a weight's current values for the derived-copy caches
    below: its version counter, which every in-place update bumps.  Tensors
    made under torch.inference_mode have no version counter; for them the key
    is the storage address and layout, so an in-place update of such a weight
    must be followed by drop_derived(w)."""
    try:
        return ("version", w._version)
    except RuntimeError:
        return ("storage", w.data_ptr(), tuple(w.shape), tuple(w.stride()))


def drop_derived(w: torch.Tensor) -> None:
    """Forget every derived copy made from ``w`` (the transposed, padded and
    packed ones; needed only after an in-place update of an inference-mode
    weight)."""
    for a in [a for a in vars(w) if a.startswith(_DERIVED_PREFIX)]:
        delattr(w, a)


def _derived(w: torch.Tensor, attr: str, make):
    """The copy of ``w`` that ``make`` builds, made once and kept on the weight
    tensor itself (so it lives exactly as long) and remade when the weight
    changes.  Making it launches device work, which must not be recorded into
    a captured HIP graph: a capture that finds no current copy raises, and the
    caller derives the copies before capturing (``Mamba3.pack_products``)."""
    key = _weight_key(w)
    hit = getattr(w, attr, None)
    if hit is None or hit[0] != key:
        if w.is_cuda and torch.cuda.is_current_stream_capturing():
            raise _lib.MambaHipError(f"{attr[1:]}: the weight copy must be made before HIP graph capture")
        hit = (key, make(w))
        setattr(w, attr, hit)
    return hit[1]


def prefill_mm(x2d: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x2d [M, d_in] @ w [d_in, d_out] (Burn's Linear layout) for prefill-sized M.
    The product runs on a [d_out, d_in] contiguous copy of w through its
    transposed view: hipBLASLt's kernels for that layout measured 9-19 % faster
    at the 2.7B-layer shapes.  The copy is made once per weight and kept on the
    weight tensor itself, remade when the weight is updated in place; it
    doubles that weight's memory for callers that prefill."""
    wt = _derived(w, "_mamba_prefill_wt", lambda t: t.t().contiguous())
    return torch.mm(x2d, wt.t())


def prefill_mm_rows(x2d: torch.Tensor, w: torch.Tensor, align: int = 8) -> torch.Tensor:
    """prefill_mm with each output row padded to a multiple of `align`
    elements: the [M, d_out] view of an [M, d_pad] product whose weight copy
    carries d_pad - d_out zero rows, so that every row of the result starts
    16-byte aligned (the vector loads of the Mamba-3 prologue kernels need it).
    Equal to prefill_mm when d_out is already a multiple of `align`."""
    d_out = w.shape[1]
    d_pad = -(-d_out // align) * align
    if d_pad == d_out:
        return prefill_mm(x2d, w)
    wt = _derived(w, "_mamba_prefill_wt_pad",
                  lambda t: torch.cat([t.t(), t.new_zeros((d_pad - d_out, t.shape[0]))]).contiguous())
    return torch.mm(x2d, wt.t())[:, :d_out]


def batch_parts(b: int, max_parts: int) -> int:
    """Row parts of the batch-split decode schedule for a batch of ``b`` rows:
    1 (one stream) below 34 rows or above 256, else ceil(b / 32) parts (at
    most 32 rows each, one MFMA row tile of the weight-streaming products), at
    least 2 and at most ``max_parts``.  Parts are independent row ranges of
    the batch stepped on their own streams: one part's latency-bound products
    overlap another's bandwidth-bound state kernel, and every part reads the
    weights once, which is what ``max_parts`` trades against."""
    if not 34 <= b <= 256:
        return 1
    return max(2, min(max_parts, -(-b // 32)))


def step_mm(x2d: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None,
            workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x2d [rows, d_in] @ w [d_in, d_out] for decode-sized rows (<= 256) through
    mamba_linear_fwd on a packed copy of w, made once and kept on the weight
    tensor (remade after an in-place update).  Measured faster than hipBLASLt's
    skinny products at the Mamba-3 block shapes; `out` f32 (default) or bf16.
    The packed operands are bf16, so w must be bf16 (an f32 weight would be
    rounded), and d_in a multiple of 16 with x2d's rows contiguous."""
    return linear(x2d, packed_weight(w), w.shape[1], out=out, workspace=workspace)


def packed_weight(w: torch.Tensor) -> torch.Tensor:
    """The packed copy of a bf16 Linear weight that step_mm streams, made once
    and kept on the weight tensor (remade after an in-place update)."""
    if w.dtype != torch.bfloat16:
        raise _lib.MambaHipError("step_mm packs bf16 weights only")
    return _derived(w, "_mamba_packed", pack_linear)


def step_mm_ok(x2d: torch.Tensor, w: torch.Tensor) -> bool:
    """True where step_mm applies: a bf16 weight whose d_in is a multiple of
    16, at most 256 rows and a unit inner stride of x2d."""
    return (w.dtype == torch.bfloat16 and x2d.dim() == 2 and x2d.shape[0] <= 256 and x2d.stride(1) == 1
            and w.shape[0] % 16 == 0)


def div_eps(dtype: torch.dtype) -> float:
    """div_eps (src/utils/mod.rs:50-95) of the reference's tensor dtype."""
    return {torch.float64: 4.0693917e-16, torch.float32: 8.1584695e-8, torch.float16: 7.1209995e-4,
            torch.bfloat16: 2.0885676e-5}[dtype]


def conv_fwd(cfg: Mamba2Config, zxbcdt: torch.Tensor, cache: Mamba2Cache, conv_w, conv_b, dt_bias,
             io_dtype=None):
    """mamba2_conv_fwd (Mamba2::forward steps 2 and 4, src/mamba2/mamba2.rs:618-699):
    zxbcdt [b, l, d_in_proj] (unit inner stride) -> (xbc [b, l, conv_dim], dt [b, l, nheads] f32).
    cache.conv_bvk is updated in place."""
    b, L, row = zxbcdt.shape
    if row != cfg.d_in_proj or zxbcdt.stride(2) != 1:
        raise _lib.MambaHipError(f"zxbcdt must be [b, l, {cfg.d_in_proj}] with a unit inner stride")
    dev = zxbcdt.device
    xbc = torch.empty((b, L, cfg.conv_dim), device=dev, dtype=io_dtype or zxbcdt.dtype)
    dt = torch.empty((b, L, cfg.nheads), device=dev, dtype=torch.float32)
    cs = cache.conv_bvk
    if cs.dtype != torch.float32 or not cs.is_contiguous() or tuple(cs.shape) != (b, cfg.conv_dim, cfg.conv_kernel):
        raise _lib.MambaHipError("conv_bvk must be a contiguous f32 [b, conv_dim, conv_kernel] tensor")
    a = _lib.Mamba2ConvArgs()
    a.batch, a.seqlen, a.channels, a.kernel, a.nheads = b, L, cfg.conv_dim, cfg.conv_kernel, cfg.nheads
    a.in_dtype, a.out_dtype = _dtype_code(zxbcdt), _dtype_code(xbc)
    a.proj, a.proj_sb, a.proj_sl = zxbcdt.data_ptr(), zxbcdt.stride(0), zxbcdt.stride(1)
    a.xbc_offset, a.dt_offset = cfg.d_inner, cfg.d_inner + cfg.conv_dim
    # converted copies held until the launch is queued
    w, bias, dtb = (None if t is None else t.contiguous().float() for t in (conv_w, conv_b, dt_bias))
    a.conv_w = w.data_ptr()
    a.conv_b = None if bias is None else bias.data_ptr()
    a.conv_state = cs.data_ptr()
    a.dt_bias = dtb.data_ptr()
    a.dt_min, a.dt_max = cfg.dt_limit
    a.xbc, a.xbc_sb, a.xbc_sl = xbc.data_ptr(), xbc.stride(0), xbc.stride(1)
    a.dt = dt.data_ptr()
    check(_lib.lib().mamba2_conv_fwd(ctypes.byref(a), _stream(dev)), "mamba2_conv_fwd")
    return xbc, dt


def gated_rmsnorm(y: torch.Tensor, z: torch.Tensor, gamma: torch.Tensor, eps: Optional[float] = None,
                  norm_before_gate: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """mamba2_gated_rmsnorm (RmsNormGated::forward, src/modules/norm/rms_norm_gated.rs:70-135):
    y, z [b, l, width] (unit inner stride) -> [b, l, width] in y's dtype.  eps defaults
    to div_eps of y's dtype, as the reference computes in that dtype."""
    b, L, W = y.shape
    if tuple(z.shape) != (b, L, W) or y.stride(2) != 1 or z.stride(2) != 1:
        raise _lib.MambaHipError("y and z must be [b, l, width] with a unit inner stride")
    if out is None:
        out = torch.empty((b, L, W), device=y.device, dtype=y.dtype)
    g = gamma.contiguous().float()
    a = _lib.Mamba2GatedNormArgs()
    a.batch, a.seqlen, a.width, a.norm_before_gate = b, L, W, int(bool(norm_before_gate))
    a.y_dtype, a.z_dtype, a.out_dtype = _dtype_code(y), _dtype_code(z), _dtype_code(out)
    a.eps = div_eps(y.dtype) if eps is None else eps
    a.y, a.y_sb, a.y_sl = y.data_ptr(), y.stride(0), y.stride(1)
    a.z, a.z_sb, a.z_sl = z.data_ptr(), z.stride(0), z.stride(1)
    a.gamma = g.data_ptr()
    a.out, a.out_sb, a.out_sl = out.data_ptr(), out.stride(0), out.stride(1)
    check(_lib.lib().mamba2_gated_rmsnorm(ctypes.byref(a), _stream(y.device)), "mamba2_gated_rmsnorm")
    return out


@dataclass
class Mamba2:
    """Mamba2 block (parameters of src/mamba2/mamba2.rs:391-505): the prefill
    forward and the decode step."""
    cfg: Mamba2Config
    in_proj_w: torch.Tensor            # [d_model, d_in_proj]
    in_proj_b: Optional[torch.Tensor]
    conv_w: torch.Tensor               # [conv_dim, conv_kernel] f32
    conv_b: Optional[torch.Tensor]     # [conv_dim] f32
    dt_bias: torch.Tensor              # [nheads] f32
    a_log: torch.Tensor                # [nheads] f32
    d: torch.Tensor                    # [nheads] f32
    norm_w: torch.Tensor               # [d_inner] f32
    out_proj_w: torch.Tensor           # [d_inner, d_model]
    out_proj_b: Optional[torch.Tensor]
    A: torch.Tensor = field(init=False, repr=False)   # [nheads] f32, -exp(a_log)

    def __post_init__(self):
        # A = -exp(a_log) (mamba2.rs:929), computed once at construction so that
        # a captured step never allocates it
        self.A = -torch.exp(self.a_log)

    @property
    def dtype(self):
        return self.in_proj_w.dtype

    def new_cache(self, batch: int) -> Mamba2Cache:
        c = self.cfg
        dev = self.in_proj_w.device
        return Mamba2Cache(
            conv_bvk=torch.zeros(batch, c.conv_dim, c.conv_kernel, device=dev, dtype=torch.float32),
            ssm_bhpr=torch.zeros(batch, c.nheads, c.per_head_dim, c.state_rank, device=dev, dtype=torch.float32))

    def forward(self, input_bsm: torch.Tensor, cache: Optional[Mamba2Cache] = None,
                chunk_len: Optional[int] = None, init_state_hpr: Optional[torch.Tensor] = None,
                events: Optional[list] = None):
        """Mamba2::forward (src/mamba2/mamba2.rs:546-786): input [b, s, d_model] ->
        (out [b, s, d_model], cache).  in_proj and out_proj are library GEMMs;
        the conv prologue (mamba2_conv_fwd), the SSD (mamba_ssd2_fwd on strided
        views of the conv output, B/C in group form) and the gated RMSNorm
        (mamba2_gated_rmsnorm) are this library's kernels.  chunk_len None is
        the reference's optimal chunk (ssd_path.rs:20-163).  The cache is
        updated: conv window in place, the SSM state replaced.

        events: if a list, a timing event is recorded on the current stream
        before the first phase and after each phase, and appended as (phase,
        event) with phase in start, in_proj, conv, ssd, norm, out_proj."""
        from .ssd import ssd2_fwd

        def mark(phase):
            if events is not None:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record()
                events.append((phase, ev))

        c = self.cfg
        b, L, _ = input_bsm.shape
        if cache is None:
            cache = self.new_cache(b)
        x = input_bsm.to(self.dtype)
        mark("start")
        zxbcdt = prefill_mm(x.reshape(b * L, -1), self.in_proj_w).reshape(b, L, -1)
        if self.in_proj_b is not None:
            zxbcdt = zxbcdt + self.in_proj_b
        mark("in_proj")
        xbc, dt = conv_fwd(c, zxbcdt, cache, self.conv_w, self.conv_b, self.dt_bias)
        mark("conv")
        H, P, G, N, di = c.nheads, c.per_head_dim, c.ngroups, c.state_rank, c.d_inner
        xs = xbc[:, :, :di].unflatten(2, (H, P))
        Bm = xbc[:, :, di:di + G * N].unflatten(2, (G, N))
        Cm = xbc[:, :, di + G * N:].unflatten(2, (G, N))
        y, hT = ssd2_fwd(xs, dt, self.A, Bm, Cm, self.d, cache.ssm_bhpr, init_state_hpr, chunk_len=chunk_len)
        cache.ssm_bhpr = hT
        mark("ssd")
        yn = gated_rmsnorm(y.flatten(2), zxbcdt[:, :, :di], self.norm_w, norm_before_gate=c.is_norm_before_gate)
        mark("norm")
        out = prefill_mm(yn.reshape(b * L, -1), self.out_proj_w).reshape(b, L, -1)
        if self.out_proj_b is not None:
            out = out + self.out_proj_b
        mark("out_proj")
        return out, cache

    def step_into(self, x: torch.Tensor, cache: Mamba2Cache, zx: torch.Tensor, y: torch.Tensor,
                  out: torch.Tensor, workspace: torch.Tensor, events=None):
        """Allocation-free step: x [b, d_model] (weight dtype) -> out [b, d_model]; cache updated in place."""
        torch.mm(x, self.in_proj_w, out=zx)
        if self.in_proj_b is not None:
            zx.add_(self.in_proj_b)
        args = step_ssm_args(self.cfg, zx, cache, self.conv_w, self.conv_b, self.dt_bias, self.A, self.d,
                             self.norm_w, y)
        step_ssm(args, workspace, events)
        torch.mm(y, self.out_proj_w, out=out)
        if self.out_proj_b is not None:
            out.add_(self.out_proj_b)

    def step(self, input_bm: torch.Tensor, cache: Optional[Mamba2Cache] = None):
        """Mamba2::step (mamba2.rs:820-1004): returns (out_bm, cache); the cache is updated in place."""
        b = input_bm.shape[0]
        if cache is None:
            cache = self.new_cache(b)
        dev, dt = input_bm.device, self.dtype
        zx = torch.empty(b, self.cfg.d_in_proj, device=dev, dtype=dt)
        y = torch.empty(b, self.cfg.d_inner, device=dev, dtype=dt)
        out = torch.empty(b, self.cfg.d_model, device=dev, dtype=dt)
        args = step_ssm_args(self.cfg, zx, cache, self.conv_w, self.conv_b, self.dt_bias, self.A, self.d,
                             self.norm_w, y)
        ws = torch.empty(_lib.lib().mamba2_step_workspace_size(ctypes.byref(args)), device=dev, dtype=torch.uint8)
        self.step_into(input_bm.to(dt), cache, zx, y, out, ws)
        return out, cache


@dataclass
class Mamba2Layer:
    """Pre-norm residual layer (src/modules/layer.rs:224-232) around a Mamba2 block."""
    norm_w: torch.Tensor   # [d_model] f32 RmsNorm gamma
    mixer: Mamba2


class Mamba2Stack:
    """A stack of pre-norm Mamba2 layers stepped one token at a time.

    The residual stream is kept in f32.  With ``fused`` (the default where the
    shape allows: headdim 64, dstate 64/128, conv width 4, batch <= 256) the
    whole stack is one mamba2_stack_step call: per layer four kernels (in_proj,
    state update, out_proj, and a per-row pass doing the residual, the gated
    norm's 1/rms, the B/C window slide and the next layer's pre-norm) on
    weights packed once at construction.  Otherwise the residual add of layer l is fused with the
    RmsNorm of layer l+1 (one mamba_rmsnorm call) around torch.mm products and
    mamba2_step_ssm.  All activations live in buffers allocated once per batch
    size, so ``step_`` allocates nothing and can be captured in a HIP graph.
    With ``split_batch`` (the default), a fused step of a batch of 34 to 256
    rows runs as two row parts (halves) on two streams (``parts``,
    ``batch_parts``): the rows never interact, and one half's weight-streaming
    products overlap the other half's state kernel (each half reads the
    weights once).  From 34 rows on, one stream would run the products on two
    32-row tiles while the halves run on one each; at 32 rows and below the
    schedule measured slower."""

    def __init__(self, layers: List[Mamba2Layer], fused: bool = True, split_batch: bool = True):
        assert layers
        self.layers = layers
        self.cfg = layers[0].mixer.cfg
        self._bufs = {}
        self._args = {}
        self.split_batch = split_batch
        self._side = None  # the streams of the batch-split schedule, made on first use
        c = self.cfg
        self.fused = fused and c.per_head_dim == 64 and c.state_rank in (64, 128) and c.conv_kernel == 4 \
            and c.d_model % 16 == 0 and c.d_model <= 4096 and c.nheads <= 256
        # packed in_proj / out_proj per layer (mamba_linear_pack), built once
        self._packed = [(pack_linear(l.mixer.in_proj_w), pack_linear(l.mixer.out_proj_w)) for l in layers] \
            if self.fused else None
        self._bias_f32 = [tuple(None if t is None else t.float().contiguous()
                                for t in (l.mixer.in_proj_b, l.mixer.out_proj_b)) for l in layers]

    @staticmethod
    def init(cfg: Mamba2Config, n_layers: int, device, dtype=torch.bfloat16,
             generator: Optional[torch.Generator] = None, fused: bool = True) -> "Mamba2Stack":
        return Mamba2Stack([Mamba2Layer(norm_w=torch.ones(cfg.d_model, device=device, dtype=torch.float32),
                                        mixer=cfg.init(device, dtype, generator)) for _ in range(n_layers)],
                           fused=fused)

    def _layer_args(self, i: int, x_res: torch.Tensor, cache: Mamba2Cache, concurrent: bool = False) -> Mamba2LayerArgs:
        key = (i, x_res.data_ptr(), x_res.shape[0], x_res.stride(0), cache.conv_bvk.data_ptr(),
               cache.ssm_bhpr.data_ptr(), concurrent)
        a = self._args.get(key)
        if a is not None:
            return a
        c, m = self.cfg, self.layers[i].mixer
        b = x_res.shape[0]
        if tuple(cache.ssm_bhpr.shape) != (b, c.nheads, c.per_head_dim, c.state_rank) or \
                tuple(cache.conv_bvk.shape) != (b, c.conv_dim, c.conv_kernel):
            raise _lib.MambaHipError("cache shapes do not match the config / batch")
        a = Mamba2LayerArgs()
        a.batch, a.d_model, a.nheads, a.headdim = b, c.d_model, c.nheads, c.per_head_dim
        a.ngroups, a.dstate, a.conv_kernel = c.ngroups, c.state_rank, c.conv_kernel
        a.norm_before_gate = int(c.is_norm_before_gate)
        a.zxbcdt_dtype = _lib.MAMBA_BF16 if m.dtype == torch.bfloat16 else _lib.MAMBA_F32
        a.x, a.x_sb = x_res.data_ptr(), x_res.stride(0)
        a.pre_norm_w = self.layers[i].norm_w.data_ptr()
        a.in_proj, a.out_proj = self._packed[i][0].data_ptr(), self._packed[i][1].data_ptr()
        ib, ob = self._bias_f32[i]
        a.in_proj_b = None if ib is None else ib.data_ptr()
        a.out_proj_b = None if ob is None else ob.data_ptr()
        a.conv_state, a.conv_w = cache.conv_bvk.data_ptr(), m.conv_w.data_ptr()
        a.conv_b = None if m.conv_b is None else m.conv_b.data_ptr()
        a.dt_bias, a.A, a.D = m.dt_bias.data_ptr(), m.A.data_ptr(), m.d.data_ptr()
        a.dt_min, a.dt_max = float(c.dt_limit[0]), float(c.dt_limit[1])
        a.norm_w, a.ssm_state = m.norm_w.data_ptr(), cache.ssm_bhpr.data_ptr()
        a.concurrent = int(concurrent)
        self._args[key] = a
        return a

    def new_caches(self, batch: int) -> List[Mamba2Cache]:
        return [l.mixer.new_cache(batch) for l in self.layers]

    def buffers(self, batch: int, device, slot: int = 0):
        key = (batch, str(device), slot)
        if key not in self._bufs:
            c, dt = self.cfg, self.layers[0].mixer.dtype
            bufs = dict(
                normed=torch.empty(batch, c.d_model, device=device, dtype=dt),
                zx=torch.empty(batch, c.d_in_proj, device=device, dtype=dt),
                y=torch.empty(batch, c.d_inner, device=device, dtype=dt),
                out=torch.empty(batch, c.d_model, device=device, dtype=dt))
            probe = Mamba2StepArgs()
            probe.batch, probe.nheads, probe.headdim = batch, c.nheads, c.per_head_dim
            n = _lib.lib().mamba2_step_workspace_size(ctypes.byref(probe))
            if self.fused:
                la = Mamba2LayerArgs()
                la.batch, la.d_model, la.nheads, la.headdim = batch, c.d_model, c.nheads, c.per_head_dim
                la.ngroups, la.dstate, la.conv_kernel = c.ngroups, c.state_rank, c.conv_kernel
                la.zxbcdt_dtype = _lib.MAMBA_BF16 if dt == torch.bfloat16 else _lib.MAMBA_F32
                for la.concurrent in (0, 1):
                    n = max(n, _lib.lib().mamba2_layer_workspace_size(ctypes.byref(la)))
            bufs["ws"] = torch.empty(n, device=device, dtype=torch.uint8)
            self._bufs[key] = bufs
        return self._bufs[key]

    # Streams of the batch-split schedule.  Each part reads every layer's
    # weights once, and this stack's weights are large next to its caches:
    # at 96 / 128 rows three or four parts measured 8.09 -> 8.32 ms and
    # 9.99 -> 10.77 ms per 64-layer step against two, at 256 rows four tied
    # with two and eight lost.
    max_parts = 2

    def parts(self, b: int) -> int:
        """Row parts of an untimed step of batch ``b``, each on its own stream (batch_parts)."""
        return batch_parts(b, self.max_parts) if (self.fused and self.split_batch) else 1

    def splits(self, b: int) -> bool:
        """Whether an untimed step of batch ``b`` runs as row parts on several streams."""
        return self.parts(b) > 1

    def step_(self, x_res: torch.Tensor, caches: List[Mamba2Cache], events=None):
        """In-place step of the whole stack: x_res [b, d_model] f32 becomes the stack output.

        ``events``: optional list of one torch.cuda.Event pair per layer,
        recorded around that layer's state-update kernel (benchmark timing)."""
        b = x_res.shape[0]
        K = self.parts(b) if events is None else 1
        if K > 1 and x_res.data_ptr() % 16 == 0 and x_res.stride(0) % 4 == 0 and x_res.is_cuda:
            # independent row parts on K streams: one part's weight-streaming products
            # run while another's state kernel streams the caches (each part reads the
            # weights once; rows never interact, so the step is the same)
            cur = torch.cuda.current_stream(x_res.device)
            if self._side is None or len(self._side) < K:
                self._side = tuple(torch.cuda.Stream(x_res.device) for _ in range(K))
            bounds = [(b * k) // K for k in range(K + 1)]
            for k in range(K):
                lo, hi = bounds[k], bounds[k + 1]
                st = self._side[k]
                st.wait_stream(cur)
                with torch.cuda.stream(st):
                    part = [Mamba2Cache(conv_bvk=cc.conv_bvk[lo:hi], ssm_bhpr=cc.ssm_bhpr[lo:hi]) for cc in caches]
                    self._stack_fused(x_res[lo:hi], part, None, slot=1 + k)
            for st in self._side[:K]:
                cur.wait_stream(st)
            return x_res
        bufs = self.buffers(b, x_res.device)
        if self.fused and b <= 256 and x_res.data_ptr() % 16 == 0 and x_res.stride(0) % 4 == 0:
            return self._stack_fused(x_res, caches, events)
        prev = None
        for i, layer in enumerate(self.layers):
            rmsnorm(x_res, layer.norm_w, out=bufs["normed"], add=prev)
            layer.mixer.step_into(bufs["normed"], caches[i], bufs["zx"], bufs["y"], bufs["out"], bufs["ws"],
                                  None if events is None else events[i])
            prev = bufs["out"]
        rmsnorm(x_res, None, add=prev)
        return x_res

    def _stack_fused(self, x_res: torch.Tensor, caches: List[Mamba2Cache], events, slot: int = 0):
        """The whole stack as one mamba2_stack_step call on the current stream."""
        bufs = self.buffers(x_res.shape[0], x_res.device, slot)
        L = _lib.lib()
        ws = bufs["ws"]
        wsp, stream = ctypes.c_void_p(ws.data_ptr()), _stream(x_res.device)
        # every pointer the per-layer args embed (the residual row and both caches);
        # slots 1 .. K are the row parts of the batch-split schedule (concurrent calls)
        concurrent = slot > 0
        key = ("stack", x_res.data_ptr(), x_res.shape[0], x_res.stride(0), concurrent) + tuple(
            (c.conv_bvk.data_ptr(), c.ssm_bhpr.data_ptr()) for c in caches)
        arr = self._args.get(key)
        if arr is None:
            arr = (Mamba2LayerArgs * len(self.layers))(
                *[self._layer_args(i, x_res, caches[i], concurrent) for i in range(len(self.layers))])
            self._args[key] = arr
        if events is None:
            check(L.mamba2_stack_step(arr, len(self.layers), wsp, ws.numel(), stream), "mamba2_stack_step")
        else:
            raw = [_raw_events(ev, x_res.device) for ev in events]
            e0 = (ctypes.c_void_p * len(raw))(*[r[0] for r in raw])
            e1 = (ctypes.c_void_p * len(raw))(*[r[1] for r in raw])
            check(L.mamba2_stack_step_timed(arr, len(self.layers), wsp, ws.numel(), stream, e0, e1),
                  "mamba2_stack_step_timed")
        return x_res

    def step(self, x: torch.Tensor, caches: Optional[List[Mamba2Cache]] = None):
        """Out-of-place convenience: returns (y [b, d_model] f32, caches)."""
        if caches is None:
            caches = self.new_caches(x.shape[0])
        x_res = x.to(torch.float32).clone()
        self.step_(x_res, caches)
        return x_res, caches
