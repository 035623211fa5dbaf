"""Mamba-3 SSD host interfaces over the C ABI: the single-pass SSD
(``mamba_ssd3_fwd``) and the double-SSD seam (``mamba_ssd3_double_fwd``).

References: ``Mamba3SingleSsdInput`` / ``run`` (src/mamba3/single_ssd/ssd/ssd_path/mod.rs:25-133)
and ``Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated``
(src/mamba3/single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-164);
``Mamba3DoubleSsdInput`` (src/mamba3/double_ssd/ssd/ssd_path/mod.rs) and
``Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated``
(src/mamba3/double_ssd/ssd/serial_recalculated/serial_recalculated.rs:76-94).
The reference's chunked [b, n, l, ...] tensors are the [b, n*l, ...] tensors
here with chunk_len = l.  Tensors are PyTorch device tensors used as memory.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import Ssd3Args, Ssd3BwdArgs, Ssd3DoubleArgs, check
from .ssd import _dtype_code, _raw_events, _stream, workspace


def _args(v, da, B, C, gamma, scale, initial_state, chunk_len, y, final_state) -> Ssd3Args:
    b, l, m, h, p = v.shape
    g, n = B.shape[3], B.shape[4]
    if B.shape != C.shape or B.shape[:3] != (b, l, m):
        raise _lib.MambaHipError("B and C must be [b, l, m, g, n] matching v")
    for t, nm in ((v, "v"), (B, "B"), (C, "C")):
        if t.stride(-1) != 1:
            raise _lib.MambaHipError(f"{nm}: innermost axis must be contiguous")
    for t, nm in ((da, "da"), (gamma, "gamma"), (scale, "scale")):
        if t.dtype != torch.float32 or t.shape != (b, l, h):
            raise _lib.MambaHipError(f"{nm} must be float32 [b, l, h]")
    for t in (initial_state, final_state):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise _lib.MambaHipError("states must be contiguous float32")
    a = Ssd3Args()
    a.batch, a.seqlen, a.mimo, a.nheads, a.headdim, a.ngroups, a.dstate = b, l, m, h, p, g, n
    a.chunk_len, a.io_dtype = int(chunk_len), _dtype_code(v)
    a.v = v.data_ptr(); a.v_sb, a.v_sl, a.v_sm, a.v_sh = v.stride()[:4]
    a.da = da.data_ptr(); a.da_sb, a.da_sl, a.da_sh = da.stride()
    a.gamma = gamma.data_ptr(); a.gamma_sb, a.gamma_sl, a.gamma_sh = gamma.stride()
    a.scale = scale.data_ptr(); a.scale_sb, a.scale_sl, a.scale_sh = scale.stride()
    a.B = B.data_ptr(); a.B_sb, a.B_sl, a.B_sm, a.B_sg = B.stride()[:4]
    a.C = C.data_ptr(); a.C_sb, a.C_sl, a.C_sm, a.C_sg = C.stride()[:4]
    a.initial_state = None if initial_state is None else initial_state.data_ptr()
    a.y = y.data_ptr(); a.y_sb, a.y_sl, a.y_sm, a.y_sh = y.stride()[:4]
    a.final_state = final_state.data_ptr()
    return a


def _outputs(v, B, y, final_state):
    b, l, m, h, p = v.shape
    if y is None:
        y = torch.empty((b, l, m, h, p), dtype=v.dtype, device=v.device)
    if final_state is None:
        final_state = torch.empty((b, h, p, B.shape[4]), dtype=torch.float32, device=v.device)
    return y, final_state


def ssd3_fast_path(v, da, B, C, gamma, scale, chunk_len=64) -> bool:
    """True when ``ssd3_fwd`` takes the single-kernel MFMA path for these tensors."""
    y, hT = _outputs(v, B, None, None)
    a = _args(v, da, B, C, gamma, scale, None, chunk_len, y, hT)
    r = _lib.lib().mamba_ssd3_fast_path(ctypes.byref(a))
    if r < 0:
        check(1, "mamba_ssd3_fast_path")
    return r == 1


def ssd3_fwd(v, da, B, C, gamma, scale, initial_state=None, chunk_len=64, y=None, final_state=None,
             events=None, generic=False):
    """v [b, l, m, h, p]; da, gamma, scale [b, l, h] f32; B, C [b, l, m, g, n] (g = h for
    per-head B/C); initial_state [b, h, p, n] f32.  Returns (y [b, l, m, h, p], final_state).
    ``generic`` forces the shape-generic kernels (cross-checks of the fast path)."""
    y, final_state = _outputs(v, B, y, final_state)
    a = _args(v, da, B, C, gamma, scale, initial_state, chunk_len, y, final_state)
    L = _lib.lib()
    need = L.mamba_ssd3_workspace_size(ctypes.byref(a))
    if need == 0:
        # invalid arguments: the call reports why
        check(L.mamba_ssd3_fwd(ctypes.byref(a), None, 0, _stream(v.device)), "mamba_ssd3_fwd")
    ws = workspace(v.device, need)
    st, wsp = _stream(v.device), ctypes.c_void_p(ws.data_ptr())
    if events is not None:
        if generic:
            raise _lib.MambaHipError("events time the default path only")
        e0, e1 = _raw_events(events, v.device)
        check(L.mamba_ssd3_fwd_timed(ctypes.byref(a), wsp, ws.numel(), st, e0, e1), "mamba_ssd3_fwd_timed")
    elif generic:
        check(L.mamba_ssd3_fwd_generic(ctypes.byref(a), wsp, ws.numel(), st), "mamba_ssd3_fwd_generic")
    else:
        check(L.mamba_ssd3_fwd(ctypes.byref(a), wsp, ws.numel(), st), "mamba_ssd3_fwd")
    return y, final_state


@dataclass
class Mamba3SingleSsdInput:
    """The reference's input bundle with [b, l, ...] tensors (the chunk axis folded into l).

    ``init_state_hpr`` (the learnable initial state) is added to
    ``initial_state_bhpr``; ``siso_specialization`` is a reference-side
    performance switch with no effect on the result."""
    v_blmhp: torch.Tensor
    b_blmhr: torch.Tensor
    c_blmhr: torch.Tensor
    da_blh: torch.Tensor
    gamma_blh: torch.Tensor
    scale_blh: torch.Tensor
    initial_state_bhpr: Optional[torch.Tensor] = None
    init_state_hpr: Optional[torch.Tensor] = None
    siso_specialization: bool = False

    def run(self, chunk_len: int = 64):
        h0 = self.initial_state_bhpr
        if self.init_state_hpr is not None:
            base = h0 if h0 is not None else torch.zeros(
                (self.v_blmhp.shape[0],) + tuple(self.init_state_hpr.shape), device=self.v_blmhp.device)
            h0 = (base + self.init_state_hpr.unsqueeze(0)).contiguous()
        return ssd3_fwd(self.v_blmhp, self.da_blh, self.b_blmhr, self.c_blmhr, self.gamma_blh, self.scale_blh,
                        h0, chunk_len)


def _double_args(v, da, B, C, initial_state, chunk_len, y, final_state) -> Ssd3DoubleArgs:
    b, l, m, h, p = v.shape
    if B.shape != C.shape or B.shape[:3] != (b, l, m):
        raise _lib.MambaHipError("B and C must be [b, l, m, g, n] matching v")
    for t, nm in ((v, "v"), (B, "B"), (C, "C")):
        if t.stride(-1) != 1:
            raise _lib.MambaHipError(f"{nm}: innermost axis must be contiguous")
    if da.dtype != torch.float32 or da.shape != (b, l, h):
        raise _lib.MambaHipError("da must be float32 [b, l, h]")
    for t in (initial_state, final_state):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise _lib.MambaHipError("states must be contiguous float32")
    a = Ssd3DoubleArgs()
    a.batch, a.seqlen, a.mimo, a.nheads, a.headdim, a.ngroups, a.dstate = b, l, m, h, p, B.shape[3], B.shape[4]
    a.chunk_len, a.io_dtype = int(chunk_len), _dtype_code(v)
    a.v = v.data_ptr(); a.v_sb, a.v_sl, a.v_sm, a.v_sh = v.stride()[:4]
    a.da = da.data_ptr(); a.da_sb, a.da_sl, a.da_sh = da.stride()
    a.B = B.data_ptr(); a.B_sb, a.B_sl, a.B_sm, a.B_sg = B.stride()[:4]
    a.C = C.data_ptr(); a.C_sb, a.C_sl, a.C_sm, a.C_sg = C.stride()[:4]
    a.initial_state = None if initial_state is None else initial_state.data_ptr()
    a.y = y.data_ptr(); a.y_sb, a.y_sl, a.y_sm, a.y_sh = y.stride()[:4]
    a.final_state = final_state.data_ptr()
    return a


def ssd3_double_fast_path(v, da, B, C, chunk_len=64) -> bool:
    """True when ``ssd3_double_fwd`` takes the single-kernel MFMA path for these tensors."""
    y, hT = _outputs(v, B, None, None)
    a = _double_args(v, da, B, C, None, chunk_len, y, hT)
    r = _lib.lib().mamba_ssd3_double_fast_path(ctypes.byref(a))
    if r < 0:
        check(1, "mamba_ssd3_double_fast_path")
    return r == 1


def ssd3_double_fwd(v, da, B, C, initial_state=None, chunk_len=64, y=None, final_state=None, generic=False):
    """The double-SSD seam: v (pre-scaled) [b, l, m, h, p]; da [b, l, h] f32; B, C
    [b, l, m, g, n]; initial_state [b, h, p, n] f32.  Returns (y, final_state)
    with y[t, m] = C[t, m] . h_t, h_t = exp(da_t) h_{t-1} + sum_m' v[t, m'] (x) B[t, m'].
    ``generic`` forces the shape-generic kernels."""
    y, final_state = _outputs(v, B, y, final_state)
    a = _double_args(v, da, B, C, initial_state, chunk_len, y, final_state)
    L = _lib.lib()
    st = _stream(v.device)
    need = L.mamba_ssd3_double_workspace_size(ctypes.byref(a))
    if need == 0:
        # invalid arguments: the call reports why
        check(L.mamba_ssd3_double_fwd(ctypes.byref(a), None, 0, st), "mamba_ssd3_double_fwd")
    ws = workspace(v.device, need)
    fn = L.mamba_ssd3_double_fwd_generic if generic else L.mamba_ssd3_double_fwd
    check(fn(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), st), "mamba_ssd3_double_fwd")
    return y, final_state


def ssd3_bwd(dy, v, da, B, C, gamma=None, scale=None, initial_state=None, d_final_state=None, events=None):
    """The single-SSD forward's gradients through ``mamba_ssd3_bwd``: the
    Autodiff arm of Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated
    (src/mamba3/single_ssd/ssd/serial_recalculated/backward.rs:27-299; gradient
    math combined_backward.rs:74-536).  gamma = scale = None is the double-SSD
    seam's backward (double_ssd/ssd/serial_recalculated/backward.rs:27-275).
    Inputs as ``ssd3_fwd`` (bf16 ones are read as f32), dy [b, l, m, h, p],
    d_final_state [b, h, p, n] or None.  Returns a dict of f32 gradients: dv,
    dda, dgamma / dscale (None without the weights), dB / dC [b, l, m, g, n]
    (summed over each group's heads), d_initial_state [b, h, p, n].  events:
    optional (start, stop) torch events around the reverse chunk-loop kernel."""
    b, l, m, h, p = v.shape
    g, n = B.shape[3], B.shape[4]
    f = lambda t: None if t is None else (t if t.dtype == torch.float32 else t.float())  # noqa: E731
    v, dy, B, C, da, gamma, scale, initial_state, d_final_state = map(
        f, (v, dy, B, C, da, gamma, scale, initial_state, d_final_state))
    if B.shape != C.shape or B.shape[:3] != (b, l, m) or dy.shape != v.shape:
        raise _lib.MambaHipError("B and C must be [b, l, m, g, n] and dy [b, l, m, h, p] matching v")
    for t, nm in ((v, "v"), (B, "B"), (C, "C"), (dy, "dy")):
        if t.stride(-1) != 1:
            raise _lib.MambaHipError(f"{nm}: innermost axis must be contiguous")
    for t, nm in ((da, "da"), (gamma, "gamma"), (scale, "scale")):
        if t is not None and t.shape != (b, l, h):
            raise _lib.MambaHipError(f"{nm} must be [b, l, h]")
    for t in (initial_state, d_final_state):
        if t is not None and not t.is_contiguous():
            raise _lib.MambaHipError("the states must be contiguous")
    dev = v.device
    out = dict(dv=torch.empty((b, l, m, h, p), device=dev), dda=torch.empty((b, l, h), device=dev),
               dgamma=None if gamma is None else torch.empty((b, l, h), device=dev),
               dscale=None if scale is None else torch.empty((b, l, h), device=dev),
               dB=torch.empty((b, l, m, g, n), device=dev), dC=torch.empty((b, l, m, g, n), device=dev),
               d_initial_state=torch.empty((b, h, p, n), device=dev))
    a = Ssd3BwdArgs()
    a.batch, a.seqlen, a.mimo, a.nheads, a.headdim, a.ngroups, a.dstate = b, l, m, h, p, g, n
    a.v = v.data_ptr(); a.v_sb, a.v_sl, a.v_sm, a.v_sh = v.stride()[:4]
    a.da = da.data_ptr(); a.da_sb, a.da_sl, a.da_sh = da.stride()
    if gamma is not None:
        a.gamma = gamma.data_ptr(); a.gamma_sb, a.gamma_sl, a.gamma_sh = gamma.stride()
    if scale is not None:
        a.scale = scale.data_ptr(); a.scale_sb, a.scale_sl, a.scale_sh = scale.stride()
    a.B = B.data_ptr(); a.B_sb, a.B_sl, a.B_sm, a.B_sg = B.stride()[:4]
    a.C = C.data_ptr(); a.C_sb, a.C_sl, a.C_sm, a.C_sg = C.stride()[:4]
    a.initial_state = None if initial_state is None else initial_state.data_ptr()
    a.dy = dy.data_ptr(); a.dy_sb, a.dy_sl, a.dy_sm, a.dy_sh = dy.stride()[:4]
    a.d_final_state = None if d_final_state is None else d_final_state.data_ptr()
    for k in ("dv", "dda", "dgamma", "dscale", "dB", "dC", "d_initial_state"):
        setattr(a, k, None if out[k] is None else out[k].data_ptr())
    L = _lib.lib()
    need = L.mamba_ssd3_bwd_workspace_size(ctypes.byref(a))
    st = _stream(dev)
    if need == 0:
        # invalid arguments: the call reports why
        check(L.mamba_ssd3_bwd(ctypes.byref(a), None, 0, st), "mamba_ssd3_bwd")
    ws = workspace(dev, need)
    if events is None:
        check(L.mamba_ssd3_bwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), st), "mamba_ssd3_bwd")
    else:
        e0, e1 = _raw_events(events, dev)
        check(L.mamba_ssd3_bwd_timed(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), st, e0, e1),
              "mamba_ssd3_bwd_timed")
    return out


class _Ssd3Function(torch.autograd.Function):
    """The single-SSD seam as one differentiable node: ``mamba_ssd3_fwd``
    forward, ``mamba_ssd3_bwd`` backward from the saved leaf inputs (the
    reference's Autodiff arm, single_ssd/ssd/serial_recalculated/
    backward.rs:27-299: one node for both outputs, intermediates recomputed)."""

    @staticmethod
    def forward(ctx, v, da, B, C, gamma, scale, initial_state, chunk_len):
        y, hT = ssd3_fwd(v, da, B, C, gamma, scale, initial_state, chunk_len=chunk_len)
        ctx.save_for_backward(v, da, B, C, gamma, scale, initial_state)
        return y, hT

    @staticmethod
    def backward(ctx, dy, dhT):
        v, da, B, C, gamma, scale, h0 = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros(v.shape, device=v.device)
        gr = ssd3_bwd(dy.contiguous(), v, da, B, C, gamma, scale, h0, None if dhT is None else dhT.contiguous())
        cast = lambda t, like: t.to(like.dtype)  # noqa: E731
        return (cast(gr["dv"], v), gr["dda"], cast(gr["dB"], B), cast(gr["dC"], C), gr["dgamma"], gr["dscale"],
                None if h0 is None else gr["d_initial_state"], None)


def ssd3_autograd(v, da, B, C, gamma, scale, initial_state=None, chunk_len=64):
    """``ssd3_fwd`` as a differentiable op (torch.autograd), returning
    (y, final_state); gradients flow to v, da, B, C, gamma, scale and
    initial_state through ``mamba_ssd3_bwd``."""
    return _Ssd3Function.apply(v, da, B, C, gamma, scale, initial_state, chunk_len)


@dataclass
class Mamba3DoubleSsdInput:
    """The double-SSD seam's input bundle (src/mamba3/double_ssd/ssd/ssd_path/mod.rs)
    with [b, l, ...] tensors (the chunk axis folded into l).  ``init_state_hpr``
    (the learnable initial state) is added to ``initial_state_bhpr``."""
    v_blmhp: torch.Tensor
    da_blh: torch.Tensor
    b_blmhr: torch.Tensor
    c_blmhr: torch.Tensor
    initial_state_bhpr: Optional[torch.Tensor] = None
    init_state_hpr: Optional[torch.Tensor] = None

    def run(self, chunk_len: int = 64):
        h0 = self.initial_state_bhpr
        if self.init_state_hpr is not None:
            base = h0 if h0 is not None else torch.zeros(
                (self.v_blmhp.shape[0],) + tuple(self.init_state_hpr.shape), device=self.v_blmhp.device)
            h0 = (base + self.init_state_hpr.unsqueeze(0)).contiguous()
        return ssd3_double_fwd(self.v_blmhp, self.da_blh, self.b_blmhr, self.c_blmhr, h0, chunk_len)
