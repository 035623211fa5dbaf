"""Mamba-2 SSD host interface, mirroring the reference's pluggable-SSD seam.

Reference: ``Mamba2SsdPath`` / ``Mamba2SsdInput`` / ``run``
(src/mamba2/ssd/ssd_path.rs:20-163) and the backend extension
``Mamba2BackendExt::ssd_serial_recalculated``
(src/mamba2/ssd/serial_recalculated/serial_recalculated.rs:73-156).

All three reference algorithms (Minimal, Serial, SerialRecalculated) are exact
reformulations of one function; on this backend every variant runs the same
gfx950 kernels — the variant only carries the chunk length, as in the
reference.  Tensors are PyTorch device tensors (used as plain memory).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import MAMBA_BF16, MAMBA_F32, Ssd2Args, Ssd2BwdArgs, check


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return MAMBA_F32
    if t.dtype == torch.bfloat16:
        return MAMBA_BF16
    raise _lib.MambaHipError(f"unsupported dtype {t.dtype} (f32 or bf16)")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_WS = {}


def workspace(device, nbytes: int) -> torch.Tensor:
    """A cached per-device byte buffer of at least ``nbytes`` (stream-ordered use)."""
    key = str(device)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WS[key] = buf
    return buf


def _check_inner(t: torch.Tensor, name: str):
    if t.stride(-1) != 1:
        raise _lib.MambaHipError(f"{name}: innermost axis must be contiguous")


def _ssd2_args(x, dt, A, B, C, D, initial_state, init_state_hpr, chunk_len, y, final_state):
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    for t, nm in ((x, "x"), (B, "B"), (C, "C")):
        _check_inner(t, nm)
    if not (dt.dtype == A.dtype == torch.float32):
        raise _lib.MambaHipError("dt and A must be float32")
    for t in (A, D, initial_state, init_state_hpr, final_state):
        if t is not None and not t.is_contiguous():
            raise _lib.MambaHipError("A, D and the states must be contiguous")
    a = Ssd2Args()
    a.batch, a.seqlen, a.nheads, a.headdim, a.ngroups, a.dstate = b, l, h, p, g, n
    a.chunk_len, a.io_dtype = int(chunk_len), _dtype_code(x)
    a.x = x.data_ptr(); a.x_sb, a.x_sl, a.x_sh = x.stride(0), x.stride(1), x.stride(2)
    a.dt = dt.data_ptr(); a.dt_sb, a.dt_sl, a.dt_sh = dt.stride(0), dt.stride(1), dt.stride(2)
    a.A = A.data_ptr()
    a.B = B.data_ptr(); a.B_sb, a.B_sl, a.B_sg = B.stride(0), B.stride(1), B.stride(2)
    a.C = C.data_ptr(); a.C_sb, a.C_sl, a.C_sg = C.stride(0), C.stride(1), C.stride(2)
    a.D = None if D is None else D.data_ptr()
    a.initial_state = None if initial_state is None else initial_state.data_ptr()
    a.init_state_hpr = None if init_state_hpr is None else init_state_hpr.data_ptr()
    if y is not None:
        a.y = y.data_ptr(); a.y_sb, a.y_sl, a.y_sh = y.stride(0), y.stride(1), y.stride(2)
    if final_state is not None:
        a.final_state = final_state.data_ptr()
    return a


def ssd2_fast_path(x, dt, A, B, C, chunk_len=None) -> bool:
    """True if ``mamba_ssd2_fwd`` would take the MFMA fast path for these inputs."""
    if chunk_len is None:
        chunk_len = Mamba2SsdPath.optimal_chunk_len(B.shape[3], x.shape[3])
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    hT = torch.empty((x.shape[0], x.shape[2], x.shape[3], B.shape[3]), dtype=torch.float32,
                     device=x.device)
    a = _ssd2_args(x, dt, A, B, C, None, None, None, chunk_len, y, hT)
    r = _lib.lib().mamba_ssd2_fast_path(ctypes.byref(a))
    if r < 0:
        check(1, "mamba_ssd2_fast_path")
    return r == 1


def ssd2_fwd(x, dt, A, B, C, D=None, initial_state=None, init_state_hpr=None, chunk_len=None,
             y=None, final_state=None, generic=False, events=None):
    """Mamba-2 SSD forward through ``mamba_ssd2_fwd``.

    x[b,l,h,p] (f32|bf16)  dt[b,l,h] f32  A[h] f32  B,C[b,l,g,n] (dtype of x)
    D[h] f32  initial_state[b,h,p,n] f32  init_state_hpr[h,p,n] f32.
    Any strides are accepted for the three outer axes; the innermost axis must
    be contiguous.  Returns (y[b,l,h,p] dtype of x, final_state[b,h,p,n] f32).
    ``events`` = (start, stop) torch.cuda.Event pair recorded around the
    dominant kernel (``mamba_ssd2_fwd_timed``); used by the benchmark.
    """
    b, l, h, p = x.shape
    n = B.shape[3]
    if chunk_len is None:
        chunk_len = Mamba2SsdPath.optimal_chunk_len(n, p)
    if y is None:
        y = torch.empty((b, l, h, p), dtype=x.dtype, device=x.device)
    if final_state is None:
        final_state = torch.empty((b, h, p, n), dtype=torch.float32, device=x.device)
    a = _ssd2_args(x, dt, A, B, C, D, initial_state, init_state_hpr, chunk_len, y, final_state)
    L = _lib.lib()
    nbytes = L.mamba_ssd2_workspace_size(ctypes.byref(a))
    ws = workspace(x.device, nbytes)
    wsp, st = ctypes.c_void_p(ws.data_ptr()), _stream(x.device)
    if events is not None:
        e0, e1 = _raw_events(events, x.device)
        check(L.mamba_ssd2_fwd_timed(ctypes.byref(a), wsp, ws.numel(), st, e0, e1),
              "mamba_ssd2_fwd_timed")
    else:
        fn = L.mamba_ssd2_fwd_generic if generic else L.mamba_ssd2_fwd
        check(fn(ctypes.byref(a), wsp, ws.numel(), st), "mamba_ssd2_fwd")
    return y, final_state


def ssd2_bwd(dy, x, dt, A, B, C, D=None, initial_state=None, d_final_state=None, events=None):
    """The SSD forward's gradients through ``mamba_ssd2_bwd``: the Autodiff arm
    of Mamba2BackendExt::ssd_serial_recalculated
    (src/mamba2/ssd/serial_recalculated/backward.rs:29-321; gradient math
    combined_backward.rs:126-593).  Inputs as ``ssd2_fwd`` (bf16 ones are read
    as f32), dy[b,l,h,p], d_final_state[b,h,p,n] or None.  Returns a dict of f32
    gradients: dx[b,l,h,p], ddt[b,l,h], dA[h], dB / dC[b,l,g,n] (summed over
    each group's heads), dD[h] (None without D), d_initial_state[b,h,p,n].
    events: optional (start, stop) torch events recorded around the reverse
    chunk-loop kernel (mamba_ssd2_bwd_timed)."""
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    f = lambda t: None if t is None else (t if t.dtype == torch.float32 else t.float())  # noqa: E731
    x, dy, B, C, dt, A, D, initial_state, d_final_state = map(f, (x, dy, B, C, dt, A, D, initial_state,
                                                                d_final_state))
    for t, nm in ((x, "x"), (B, "B"), (C, "C"), (dy, "dy")):
        _check_inner(t, nm)
    for t in (A, D, initial_state, d_final_state):
        if t is not None and not t.is_contiguous():
            raise _lib.MambaHipError("A, D and the states must be contiguous")
    dev = x.device
    out = dict(dx=torch.empty((b, l, h, p), device=dev), ddt=torch.empty((b, l, h), device=dev),
               dA=torch.empty(h, device=dev), dB=torch.empty((b, l, g, n), device=dev),
               dC=torch.empty((b, l, g, n), device=dev), dD=None if D is None else torch.empty(h, device=dev),
               d_initial_state=torch.empty((b, h, p, n), device=dev))
    a = Ssd2BwdArgs()
    a.batch, a.seqlen, a.nheads, a.headdim, a.ngroups, a.dstate = b, l, h, p, g, n
    a.x = x.data_ptr(); a.x_sb, a.x_sl, a.x_sh = x.stride(0), x.stride(1), x.stride(2)
    a.dt = dt.data_ptr(); a.dt_sb, a.dt_sl, a.dt_sh = dt.stride(0), dt.stride(1), dt.stride(2)
    a.A = A.data_ptr()
    a.B = B.data_ptr(); a.B_sb, a.B_sl, a.B_sg = B.stride(0), B.stride(1), B.stride(2)
    a.C = C.data_ptr(); a.C_sb, a.C_sl, a.C_sg = C.stride(0), C.stride(1), C.stride(2)
    a.D = None if D is None else D.data_ptr()
    a.initial_state = None if initial_state is None else initial_state.data_ptr()
    a.dy = dy.data_ptr(); a.dy_sb, a.dy_sl, a.dy_sh = dy.stride(0), dy.stride(1), dy.stride(2)
    a.d_final_state = None if d_final_state is None else d_final_state.data_ptr()
    for k in ("dx", "ddt", "dA", "dB", "dC", "dD"):
        setattr(a, k, None if out[k] is None else out[k].data_ptr())
    a.d_initial_state = out["d_initial_state"].data_ptr()
    L = _lib.lib()
    nbytes = L.mamba_ssd2_bwd_workspace_size(ctypes.byref(a))
    if nbytes == 0:
        check(L.mamba_ssd2_bwd(ctypes.byref(a), None, 0, _stream(dev)), "mamba_ssd2_bwd")
    ws = workspace(dev, nbytes)
    if events is None:
        check(L.mamba_ssd2_bwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(dev)),
              "mamba_ssd2_bwd")
    else:
        e0, e1 = _raw_events(events, dev)
        check(L.mamba_ssd2_bwd_timed(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(dev),
                                     e0, e1), "mamba_ssd2_bwd_timed")
    return out


class _Ssd2Function(torch.autograd.Function):
    """The SSD as one differentiable node: ``mamba_ssd2_fwd`` forward,
    ``mamba_ssd2_bwd`` backward from the saved leaf inputs (the reference's
    Autodiff arm, backward.rs:29-321: one node for both outputs, intermediates
    recomputed rather than kept)."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, D, initial_state, chunk_len):
        y, hT = ssd2_fwd(x, dt, A, B, C, D, initial_state, chunk_len=chunk_len)
        ctx.save_for_backward(x, dt, A, B, C, D, initial_state)
        return y, hT

    @staticmethod
    def backward(ctx, dy, dhT):
        x, dt, A, B, C, D, h0 = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros(x.shape, device=x.device)
        gr = ssd2_bwd(dy.contiguous(), x, dt, A, B, C, D, h0, None if dhT is None else dhT.contiguous())
        cast = lambda t, like: None if t is None else t.to(like.dtype)  # noqa: E731
        return (cast(gr["dx"], x), gr["ddt"], gr["dA"], cast(gr["dB"], B), cast(gr["dC"], C), gr["dD"],
                None if h0 is None else gr["d_initial_state"], None)


def ssd2_autograd(x, dt, A, B, C, D=None, initial_state=None, chunk_len=None):
    """``ssd2_fwd`` as a differentiable op (torch.autograd), returning
    (y, final_state); gradients flow to x, dt, A, B, C, D and initial_state
    through ``mamba_ssd2_bwd``."""
    return _Ssd2Function.apply(x, dt, A, B, C, D, initial_state, chunk_len)


def _raw_events(events, device):
    """hipEvent_t handles of a torch.cuda.Event pair (torch creates the HIP
    event lazily on first record, so record once if needed)."""
    out = []
    for e in events:
        if e.cuda_event == 0:
            e.record(torch.cuda.current_stream(device))
        out.append(ctypes.c_void_p(e.cuda_event))
    return out


class Mamba2SsdPath:
    """Algorithm selector carrying an optional chunk length (ssd_path.rs:20-53)."""

    MINIMAL, SERIAL, SERIAL_RECALCULATED = "Minimal", "Serial", "SerialRecalculated"

    def __init__(self, kind: str = SERIAL_RECALCULATED, chunk_len: Optional[int] = None):
        assert kind in (self.MINIMAL, self.SERIAL, self.SERIAL_RECALCULATED)
        self.kind, self._chunk_len = kind, chunk_len

    @staticmethod
    def optimal_chunk_len(state_rank: int, per_head_dim: int) -> int:
        """min(512, roundup32(isqrt(r*p))) — ssd_path.rs:109-114."""
        v = math.isqrt(state_rank * per_head_dim)
        v = (v + 31) // 32 * 32
        return min(v, 512)

    def chunk_len(self) -> Optional[int]:
        return self._chunk_len

    @classmethod
    def default_optimal_from_block(cls, block) -> "Mamba2SsdPath":
        """SerialRecalculated at the block's optimal chunk length (ssd_path.rs:129-134)."""
        c = block.cfg
        return cls(cls.SERIAL_RECALCULATED, cls.optimal_chunk_len(c.state_rank, c.per_head_dim))

    def chunk_len_or_optimal(self, state_rank: int, per_head_dim: int) -> int:
        return self._chunk_len if self._chunk_len is not None else self.optimal_chunk_len(
            state_rank, per_head_dim)


@dataclass
class Mamba2SsdInput:
    """Pre-processed SSD inputs in the reference's chunked shapes (ssd_path.rs:58-87).

    x_bnlhp[b,n,l,h,p]  dt_bnlh[b,n,l,h]  a_decay_h[h]  b_bnlhr/c_bnlhr[b,n,l,h,r]
    (per head, or per group with the group count in place of h)  d_h[h]
    initial_state_bhpr[b,h,p,r]  init_state_hpr[h,p,r] | None.
    """

    x_bnlhp: torch.Tensor
    dt_bnlh: torch.Tensor
    a_decay_h: torch.Tensor
    b_bnlhr: torch.Tensor
    c_bnlhr: torch.Tensor
    d_h: torch.Tensor
    initial_state_bhpr: torch.Tensor
    init_state_hpr: Optional[torch.Tensor] = None

    def run(self, path: Mamba2SsdPath):
        """Returns (y_bnlhp, final_state_bhpr) — ssd_path.rs:149-155."""
        b, nch, q, h, p = self.x_bnlhp.shape
        g, r = self.b_bnlhr.shape[3], self.b_bnlhr.shape[4]
        if nch < 1:
            raise _lib.MambaHipError("sequence length must be at least 1")
        L = nch * q
        x = self.x_bnlhp.reshape(b, L, h, p)
        dt = self.dt_bnlh.reshape(b, L, h)
        Bm = self.b_bnlhr.reshape(b, L, g, r)
        Cm = self.c_bnlhr.reshape(b, L, g, r)
        y, hT = ssd2_fwd(x, dt, self.a_decay_h, Bm, Cm, self.d_h, self.initial_state_bhpr,
                         self.init_state_hpr, chunk_len=q)
        return y.reshape(b, nch, q, h, p), hT
