"""Mamba-1 over the C ABI: the block forward (prefill conv on
``mamba2_conv_fwd`` with no dt heads, then ``mamba1_scan_fwd``), the selective
scan (``mamba1_scan_fwd``) and the recurrent decode step (``mamba1_scan_step``,
``mamba_conv1d_step``).

Reference: ``Mamba1::selective_scan`` (src/mamba1/mamba1.rs:422-523) and, with
``delta_bias``/``delta_softplus``/``z``, the scan part of ``Mamba1::ssm`` plus
the ``silu(z)`` gate of ``Mamba1::forward`` (mamba1.rs:348, 391-394); the block
``Mamba1::forward`` (mamba1.rs:278-352);
``Mamba1::step`` / ``ssm_step`` / ``selective_scan_step`` (mamba1.rs:533-733).
The x_proj / dt_proj / in_proj / out_proj products run on the ROCm BLAS
through ``torch.mm``.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib
from ._lib import Conv1dStepArgs, Mamba1ScanArgs, Mamba1StepArgs, check
from .ssd import _dtype_code, _raw_events, _stream


def _f32(t, name):
    if t is not None and t.dtype != torch.float32:
        raise _lib.MambaHipError(f"{name}: float32 required")


def mamba1_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                initial_state=None, y=None, final_state=None, events=None):
    """u, delta, z [b, d, l]; A [d, n]; B, C [b, n, l]; D, delta_bias [d];
    initial_state [b, d, n].  Any strides (u, delta, z and y sharing one stride
    pair take the tiled kernel).  Returns (y [b, d, l], final_state [b, d, n])."""
    for t, nm in ((u, "u"), (delta, "delta"), (A, "A"), (B, "B"), (C, "C"), (D, "D"), (z, "z"),
                  (delta_bias, "delta_bias"), (initial_state, "initial_state")):
        _f32(t, nm)
    b, d, l = u.shape
    n = A.shape[1]
    if y is None:
        y = torch.empty((b, d, l), dtype=torch.float32, device=u.device)
    if final_state is None:
        final_state = torch.empty((b, d, n), dtype=torch.float32, device=u.device)
    for t, nm in ((D, "D"), (delta_bias, "delta_bias"), (initial_state, "initial_state"),
                  (final_state, "final_state")):
        if t is not None and not t.is_contiguous():
            raise _lib.MambaHipError(f"{nm} must be contiguous")
    a = Mamba1ScanArgs()
    a.batch, a.dim, a.seqlen, a.dstate = b, d, l, n
    a.u = u.data_ptr(); a.u_sb, a.u_sd, a.u_sl = u.stride()
    a.delta = delta.data_ptr(); a.delta_sb, a.delta_sd, a.delta_sl = delta.stride()
    a.A = A.data_ptr(); a.A_sd, a.A_sn = A.stride()
    a.B = B.data_ptr(); a.B_sb, a.B_sn, a.B_sl = B.stride()
    a.C = C.data_ptr(); a.C_sb, a.C_sn, a.C_sl = C.stride()
    a.D = None if D is None else D.data_ptr()
    if z is not None:
        a.z = z.data_ptr(); a.z_sb, a.z_sd, a.z_sl = z.stride()
    a.delta_bias = None if delta_bias is None else delta_bias.data_ptr()
    a.delta_softplus = int(bool(delta_softplus))
    a.initial_state = None if initial_state is None else initial_state.data_ptr()
    a.y = y.data_ptr(); a.y_sb, a.y_sd, a.y_sl = y.stride()
    a.final_state = final_state.data_ptr()
    L = _lib.lib()
    st = _stream(u.device)
    if events is not None:
        e0, e1 = _raw_events(events, u.device)
        check(L.mamba1_scan_fwd_timed(ctypes.byref(a), st, e0, e1), "mamba1_scan_fwd_timed")
    else:
        check(L.mamba1_scan_fwd(ctypes.byref(a), st), "mamba1_scan_fwd")
    return y, final_state


def selective_scan(delta, a, b, c, d, u, init_ssm):
    """The reference signature and layouts (mamba1.rs:422-430):
    delta [s, b, d]; a [d, r]; b [b, s, r]; c [s, b, r]; d [d]; u [b, s, d];
    init_ssm [b, d, r]  ->  (y [b, s, d], final_state [b, d, r])."""
    s, bsz, dim = delta.shape
    # delta in u's layout so that u, delta and y share one stride pair
    delta_bsd = delta.permute(1, 0, 2).contiguous()
    y = torch.empty((bsz, s, dim), dtype=torch.float32, device=u.device)
    init = init_ssm.contiguous()
    out, hT = mamba1_scan(u.permute(0, 2, 1), delta_bsd.permute(0, 2, 1), a, b.permute(0, 2, 1),
                          c.permute(1, 2, 0), d, None, initial_state=init, y=y.permute(0, 2, 1))
    return y, hT


# --------------------------------------------------------------------------
# Recurrent decode step
# --------------------------------------------------------------------------

def scan_step(u, delta, A, B, C, state, D=None, z=None, delta_bias=None, delta_softplus=False, y=None,
              events=None):
    """mamba1_scan_step: u, delta, z [b, d]; A [d, n]; B, C [b, n] (any strides);
    state [b, d, n] contiguous f32, updated in place.  Returns y [b, d].
    ``events`` (start, stop) are recorded by the library around the kernel."""
    for t, nm in ((u, "u"), (delta, "delta"), (A, "A"), (B, "B"), (C, "C"), (D, "D"), (z, "z"),
                  (delta_bias, "delta_bias"), (state, "state")):
        _f32(t, nm)
    if not state.is_contiguous():
        raise _lib.MambaHipError("state must be contiguous")
    b, d = u.shape
    n = A.shape[1]
    if tuple(state.shape) != (b, d, n):
        raise _lib.MambaHipError(f"state shape {tuple(state.shape)} != {(b, d, n)}")
    if y is None:
        y = torch.empty((b, d), dtype=torch.float32, device=u.device)
    a = Mamba1StepArgs()
    a.batch, a.dim, a.dstate = b, d, n
    a.u, a.u_sb = u.data_ptr(), u.stride(0)
    a.delta, a.delta_sb = delta.data_ptr(), delta.stride(0)
    a.A = A.data_ptr(); a.A_sd, a.A_sn = A.stride()
    a.B = B.data_ptr(); a.B_sb, a.B_sn = B.stride()
    a.C = C.data_ptr(); a.C_sb, a.C_sn = C.stride()
    for t in (u, delta, y) + (() if z is None else (z,)):
        if t.stride(1) != 1:
            raise _lib.MambaHipError("u, delta, z and y need a contiguous channel axis")
    a.D = None if D is None else D.data_ptr()
    if z is not None:
        a.z, a.z_sb = z.data_ptr(), z.stride(0)
    a.delta_bias = None if delta_bias is None else delta_bias.data_ptr()
    a.delta_softplus = int(bool(delta_softplus))
    a.state = state.data_ptr()
    a.y, a.y_sb = y.data_ptr(), y.stride(0)
    if events is not None:
        e0, e1 = _raw_events(events, u.device)
        check(_lib.lib().mamba1_scan_step_timed(ctypes.byref(a), _stream(u.device), e0, e1),
              "mamba1_scan_step_timed")
    else:
        check(_lib.lib().mamba1_scan_step(ctypes.byref(a), _stream(u.device)), "mamba1_scan_step")
    return y


def selective_scan_step(delta, a, b, c, d, u, ssm_bir):
    """The reference signature (mamba1.rs:666-674): delta [b, d_inner]; a [d_inner, r];
    b, c [b, r]; d [d_inner]; u [b, d_inner]; the cache's ssm_bir [b, d_inner, r]
    (updated in place).  Returns (y [b, d_inner], ssm_bir)."""
    return scan_step(u, delta, a, b, c, ssm_bir, D=d), ssm_bir


def conv1d_step(x, state, w, bias=None, silu=True, out=None):
    """mamba_conv1d_step: x [b, c] (f32/bf16); state [b, c, K] f32 (in place);
    w [c, K]; bias [c].  Returns out [b, c] (f32 unless given)."""
    b, c = x.shape
    k = state.shape[2]
    if state.dtype != torch.float32 or not state.is_contiguous() or tuple(state.shape) != (b, c, k):
        raise _lib.MambaHipError("state must be a contiguous float32 [b, c, K] tensor")
    if w.dtype != torch.float32 or not w.is_contiguous() or tuple(w.shape) != (c, k):
        raise _lib.MambaHipError("w must be a contiguous float32 [c, K] tensor")
    if x.stride(1) != 1:
        raise _lib.MambaHipError("x needs a contiguous channel axis")
    if out is None:
        out = torch.empty((b, c), dtype=torch.float32, device=x.device)
    a = Conv1dStepArgs()
    a.batch, a.channels, a.kernel = b, c, k
    a.x_dtype, a.out_dtype = _dtype_code(x), _dtype_code(out)
    a.x, a.x_sb = x.data_ptr(), x.stride(0)
    a.state, a.w = state.data_ptr(), w.data_ptr()
    a.bias = None if bias is None else bias.data_ptr()
    a.silu = int(bool(silu))
    a.out, a.out_sb = out.data_ptr(), out.stride(0)
    check(_lib.lib().mamba_conv1d_step(ctypes.byref(a), _stream(x.device)), "mamba_conv1d_step")
    return out


def conv1d_fwd(x, state, w, bias=None):
    """Layer 2 of Mamba1::forward (src/mamba1/mamba1.rs:300-340) on the
    ``mamba2_conv_fwd`` kernel with no dt heads: x [b, l, c] (unit inner stride)
    -> silu(causal depthwise conv of [state[:, :, 1:] | x] + bias) [b, l, c] f32;
    state [b, c, K] (contiguous f32) becomes the last K columns of that padded
    input, in place."""
    b, L, ch = x.shape
    k = w.shape[1]
    if x.dtype != torch.float32 or x.stride(2) != 1:
        raise _lib.MambaHipError("x must be f32 with a unit inner stride")
    if state.dtype != torch.float32 or not state.is_contiguous() or tuple(state.shape) != (b, ch, k):
        raise _lib.MambaHipError("conv state must be a contiguous f32 [b, channels, K] tensor")
    out = torch.empty((b, L, ch), device=x.device, dtype=torch.float32)
    wc, bc = w.contiguous().float(), None if bias is None else bias.contiguous().float()
    a = _lib.Mamba2ConvArgs()
    a.batch, a.seqlen, a.channels, a.kernel, a.nheads = b, L, ch, k, 0
    a.in_dtype = a.out_dtype = _lib.MAMBA_F32
    a.proj, a.proj_sb, a.proj_sl = x.data_ptr(), x.stride(0), x.stride(1)
    a.xbc_offset = a.dt_offset = 0
    a.conv_w = wc.data_ptr()
    a.conv_b = None if bc is None else bc.data_ptr()
    a.conv_state = state.data_ptr()
    a.dt_bias, a.dt = None, None
    a.xbc, a.xbc_sb, a.xbc_sl = out.data_ptr(), out.stride(0), out.stride(1)
    check(_lib.lib().mamba2_conv_fwd(ctypes.byref(a), _stream(x.device)), "mamba2_conv_fwd")
    return out


@dataclass
class Mamba1Cache:
    """conv_bik [batch, d_inner, conv_kernel] and ssm_bir [batch, d_inner, state_rank], f32
    (src/mamba1/cache.rs:30-47)."""
    conv_bik: torch.Tensor
    ssm_bir: torch.Tensor


@dataclass
class Mamba1Config:
    """Mamba1Config (src/mamba1/mamba1.rs:80-123) with the reference defaults."""
    d_model: int
    state_rank: int = 16
    conv_kernel: int = 4
    expand: int = 2
    dt_min: float = 1e-3
    dt_max: float = 1e-1
    dt_scale: float = 1.0
    dt_init_floor: float = 1e-4
    has_conv_bias: bool = True
    has_proj_bias: bool = False
    dt_rank_: Optional[int] = None
    d_inner_: Optional[int] = None

    @property
    def d_inner(self) -> int:
        return self.d_inner_ or self.expand * self.d_model

    @property
    def dt_rank(self) -> int:
        return self.dt_rank_ or -(-self.d_model // self.state_rank)

    def init(self, device, generator: Optional[torch.Generator] = None) -> "Mamba1":
        """Random init following Mamba1Config::init (mamba1.rs:124-227), f32."""
        g = generator
        gdev = g.device if g is not None else torch.device("cpu")

        def rand(*shape):
            return torch.rand(shape, generator=g, device=gdev, dtype=torch.float32)

        def uni(shape, bound):
            return (rand(*shape) * 2 - 1) * bound

        di, r, n, k = self.d_inner, self.dt_rank, self.state_rank, self.conv_kernel
        lo, hi = math.log(self.dt_min), math.log(self.dt_max)
        dt = torch.exp(rand(di).double() * (hi - lo) + lo).clamp(min=self.dt_init_floor)
        f32 = dict(device=device, dtype=torch.float32)
        return Mamba1(
            cfg=self,
            in_proj_w=uni((self.d_model, 2 * di), 1 / math.sqrt(self.d_model)).to(**f32),
            conv_w=uni((di, k), 1 / math.sqrt(k)).to(**f32),
            conv_b=uni((di,), 1 / math.sqrt(k)).to(**f32) if self.has_conv_bias else None,
            x_proj_w=uni((di, r + 2 * n), 1 / math.sqrt(di)).to(**f32),
            dt_proj_w=uni((r, di), self.dt_scale / math.sqrt(r)).to(**f32),
            dt_proj_b=(dt + torch.log(-torch.expm1(-dt))).to(**f32),
            a_log=torch.log(torch.arange(1, n + 1, dtype=torch.float32)).repeat(di, 1).to(**f32),
            d=torch.ones(di, **f32),
            out_proj_w=uni((di, self.d_model), 1 / math.sqrt(di)).to(**f32),
        )


def _wt(w: torch.Tensor, attr: str, col0: int) -> torch.Tensor:
    """The contiguous transpose of w[:, col0:], made once, kept on the weight
    and remade when the weight is updated in place (the derived-copy cache of
    the decode products, mamba_hip.step)."""
    from .step import _derived
    return _derived(w, attr, lambda t: t[:, col0:].t().contiguous())


@dataclass
class Mamba1:
    """Mamba1 block, forward and step (parameters of src/mamba1/mamba1.rs:124-227);
    Linear weights in Burn's [d_in, d_out] layout."""
    cfg: Mamba1Config
    in_proj_w: torch.Tensor      # [d_model, 2 d_inner]
    conv_w: torch.Tensor         # [d_inner, K]
    conv_b: Optional[torch.Tensor]
    x_proj_w: torch.Tensor       # [d_inner, dt_rank + 2 n]
    dt_proj_w: torch.Tensor      # [dt_rank, d_inner]
    dt_proj_b: torch.Tensor      # [d_inner]
    a_log: torch.Tensor          # [d_inner, n]
    d: torch.Tensor              # [d_inner]
    out_proj_w: torch.Tensor     # [d_inner, d_model]
    A: torch.Tensor = field(init=False, repr=False)

    def __post_init__(self):
        self.A = -torch.exp(self.a_log)  # mamba1.rs:627

    def new_cache(self, batch: int) -> Mamba1Cache:
        c, dev = self.cfg, self.in_proj_w.device
        return Mamba1Cache(conv_bik=torch.zeros(batch, c.d_inner, c.conv_kernel, device=dev),
                           ssm_bir=torch.zeros(batch, c.d_inner, c.state_rank, device=dev))

    def forward(self, x: torch.Tensor, cache: Optional[Mamba1Cache] = None, events=None):
        """Mamba1::forward (src/mamba1/mamba1.rs:278-352): x [b, l, d_model] ->
        (y [b, l, d_model], cache).  The cache (zero when None) supplies the
        initial conv window and SSM state and is updated in place, so a
        sequence can be run in segments (chunked prefill, then step).
        `events` (start, stop) are recorded around the scan kernel."""
        c = self.cfg
        b, L, dm = x.shape
        if L < 1:
            raise _lib.MambaHipError("sequence length must be at least 1")
        if cache is None:
            cache = self.new_cache(b)
        di, r, n = c.d_inner, c.dt_rank, c.state_rank
        xf = x.float()
        x2 = xf.reshape(b * L, dm)
        # The scan streams u, delta, z and y as time-contiguous rows [b, d, l]
        # (its tuned kernel reads 32-token tiles of whole 128-byte lines), so
        # the products around it are formed in that layout: z and delta as
        # W^T x^T per batch row, y consumed through its transposed view.
        # layer 1, in_proj: the conv half channels-last [b, l, d_inner], the
        # gate half z time-major [b, d_inner, l]
        xs = torch.mm(x2, self.in_proj_w[:, :di]).view(b, L, di)
        zt = torch.matmul(_wt(self.in_proj_w, "_mamba_t_res", di), xf.transpose(1, 2))
        # layer 2: causal conv over [cached window | xs] + SiLU; window updated
        u = conv1d_fwd(xs, cache.conv_bik, self.conv_w, self.conv_b)
        # ssm (mamba1.rs:366-399): x_proj, dt_proj (its bias and the softplus go
        # to the scan), then the selective scan with D u and the silu(res) gate
        # (x_proj and dt_proj time-major too: B and C then stream as whole rows)
        ut = u.transpose(1, 2).contiguous()
        x_dbl = torch.matmul(_wt(self.x_proj_w, "_mamba_t", 0), ut)          # [b, r + 2n, l]
        dt = torch.matmul(_wt(self.dt_proj_w, "_mamba_t", 0), x_dbl[:, :r])  # [b, d_inner, l]
        yt = torch.empty((b, di, L), device=x.device, dtype=torch.float32)
        final = torch.empty_like(cache.ssm_bir)
        mamba1_scan(ut, dt, self.A, x_dbl[:, r:r + n], x_dbl[:, r + n:],
                    D=self.d, z=zt, delta_bias=self.dt_proj_b, delta_softplus=True,
                    initial_state=cache.ssm_bir, y=yt, final_state=final, events=events)
        cache.ssm_bir.copy_(final)
        return torch.matmul(yt.transpose(1, 2), self.out_proj_w), cache


    def step(self, x: torch.Tensor, cache: Optional[Mamba1Cache] = None):
        """Mamba1::step (mamba1.rs:533-612): returns (y [b, d_model], cache); the cache
        is updated in place."""
        c = self.cfg
        b = x.shape[0]
        if cache is None:
            cache = self.new_cache(b)
        xr = torch.mm(x.float(), self.in_proj_w)                     # [b, 2 d_inner]
        xs, res = xr[:, :c.d_inner], xr[:, c.d_inner:]
        u = conv1d_step(xs, cache.conv_bik, self.conv_w, self.conv_b, silu=True)
        x_dbl = torch.mm(u, self.x_proj_w)                           # [b, dt_rank + 2n]
        r, n = c.dt_rank, c.state_rank
        delta = torch.mm(x_dbl[:, :r], self.dt_proj_w)               # dt_proj without its bias
        y = scan_step(u, delta, self.A, x_dbl[:, r:r + n], x_dbl[:, r + n:], cache.ssm_bir, D=self.d, z=res,
                      delta_bias=self.dt_proj_b, delta_softplus=True)
        return torch.mm(y, self.out_proj_w), cache
