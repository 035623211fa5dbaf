"""Mamba-1 selective scan over the C ABI (``mamba1_scan_fwd``).

Reference: ``Mamba1::selective_scan`` (src/mamba1/mamba1.rs:422-523) and, with
``delta_bias``/``delta_softplus``/``z``, the scan part of ``Mamba1::ssm`` plus
the ``silu(z)`` gate of ``Mamba1::forward`` (mamba1.rs:348, 391-394).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import Mamba1ScanArgs, check
from .ssd import _raw_events, _stream


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
