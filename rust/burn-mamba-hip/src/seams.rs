//! The reference's SSD seams on the C ABI, independent of Burn: each function
//! takes the seam's tensors in the layouts its trait method receives them
//! (`src/mamba2/ssd/serial_recalculated/serial_recalculated.rs:86-98`,
//! `src/mamba3/single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-114`,
//! `src/mamba3/double_ssd/ssd/serial_recalculated/serial_recalculated.rs:76-94`),
//! as device pointers with element strides, maps them onto the library's
//! argument structs and calls it on `stream`.
//!
//! The chunked axes `[.., nchunks, chunk_len, ..]` of the seam are one
//! sequence axis of length `nchunks * chunk_len` for the library (they must
//! be mergeable: `stride(nchunks) == chunk_len * stride(chunk_len)`), and the
//! seam's `chunk_len` is passed as the library's chunk length.  B and C arrive
//! per head at these seams (after the reference's group expand), so the
//! library sees `ngroups = nheads` with the group stride equal to the head
//! stride.  The innermost axis of every tensor must be unit-stride.
//!
//! `workspace` returns device memory of at least the requested size (a cached
//! per-device allocation in a backend); outputs are caller-allocated.

use core::ffi::{c_int, c_void};

use crate::ffi::*;
use crate::check;

/// A device tensor: pointer, dims and element strides (rank R).
#[derive(Clone, Copy, Debug)]
pub struct Dev<const R: usize> {
    pub ptr: *mut c_void,
    pub dims: [usize; R],
    pub strides: [isize; R],
}

impl<const R: usize> Dev<R> {
    fn s(&self, i: usize) -> i64 {
        self.strides[i] as i64
    }
    fn unit_inner(&self, what: &str) {
        assert!(self.strides[R - 1] == 1 || self.dims[R - 1] == 1, "{what}: innermost axis must be unit-stride");
    }
    /// Asserts that axes (i, i + 1) merge into one axis.
    fn mergeable(&self, i: usize, what: &str) {
        assert!(
            self.dims[i] == 1 || self.strides[i] == self.dims[i + 1] as isize * self.strides[i + 1],
            "{what}: axes {i} and {} must be mergeable (nchunks x chunk_len)",
            i + 1
        );
    }
    fn contiguous(&self, what: &str) {
        let mut want = 1isize;
        for i in (0..R).rev() {
            assert!(self.dims[i] == 1 || self.strides[i] == want, "{what}: must be contiguous");
            want *= self.dims[i] as isize;
        }
    }
}

/// `Mamba2BackendExt::ssd_serial_recalculated`: x [b, n, l, h, p], dt [b, h, n, l],
/// B / C [b, n, l, h, r], D [h], initial state [b, h, p, r], A [h] (negative)
/// -> y [b, n, l, h, p] (x's layout), final state [b, h, p, r].  `io_dtype` is
/// MAMBA_F32 or MAMBA_BF16 for x, B, C and y; dt, D, A and the states are f32.
#[allow(clippy::too_many_arguments)]
pub fn ssd2_forward(
    x: Dev<5>, dt: Dev<4>, b: Dev<5>, c: Dev<5>, d: Dev<1>, h0: Dev<4>, a: Dev<1>, y: Dev<5>, hf: Dev<4>,
    io_dtype: c_int, workspace: &mut dyn FnMut(usize) -> *mut c_void, stream: MambaStream,
) {
    let [bb, n, l, h, p] = x.dims;
    let r = b.dims[4];
    for (t, w) in [(&x, "x"), (&b, "B"), (&c, "C"), (&y, "y")] {
        t.unit_inner(w);
        t.mergeable(1, w);
    }
    dt.mergeable(2, "dt");
    dt.unit_inner("dt");
    h0.contiguous("initial_state");
    hf.contiguous("final_state");
    let args = MambaSsd2Args {
        batch: bb as i32, seqlen: (n * l) as i32, nheads: h as i32, headdim: p as i32,
        ngroups: h as i32, dstate: r as i32, chunk_len: l as i32, io_dtype,
        x: x.ptr, x_sb: x.s(0), x_sl: x.s(2), x_sh: x.s(3),
        dt: dt.ptr as *const f32, dt_sb: dt.s(0), dt_sl: dt.s(3), dt_sh: dt.s(1),
        A: a.ptr as *const f32,
        B: b.ptr, B_sb: b.s(0), B_sl: b.s(2), B_sg: b.s(3),
        C: c.ptr, C_sb: c.s(0), C_sl: c.s(2), C_sg: c.s(3),
        D: d.ptr as *const f32,
        initial_state: h0.ptr as *const f32,
        init_state_hpr: core::ptr::null(),
        y: y.ptr, y_sb: y.s(0), y_sl: y.s(2), y_sh: y.s(3),
        final_state: hf.ptr as *mut f32,
    };
    // SAFETY: every pointer is a device allocation of the shape and strides
    // described above, valid on `stream` until the call's work completes.
    let bytes = unsafe { mamba_ssd2_workspace_size(&args) };
    let ws = if bytes > 0 { workspace(bytes) } else { core::ptr::null_mut() };
    check(unsafe { mamba_ssd2_fwd(&args, ws, bytes, stream) }, "mamba_ssd2_fwd");
}

/// The gradients of `ssd2_forward` (the reference's Autodiff arm,
/// `src/mamba2/ssd/serial_recalculated/backward.rs:29-321`, gradient math
/// `combined_backward.rs:126-593`), f32: from dy (y's layout) and d(final
/// state) into dx [b, n, l, h, p], ddt_blh [b, n*l, h] (position-major: the
/// seam's dt is [b, h, n, l], so the caller permutes it back), dA [h],
/// dB / dC [b, n, l, h, r], dD [h], d(initial state) [b, h, p, r], all
/// contiguous.
#[allow(clippy::too_many_arguments)]
pub fn ssd2_backward(
    x: Dev<5>, dt: Dev<4>, b: Dev<5>, c: Dev<5>, d: Dev<1>, h0: Dev<4>, a: Dev<1>, dy: Dev<5>,
    dhf: Dev<4>, dx: Dev<5>, ddt_blh: Dev<3>, da: Dev<1>, db: Dev<5>, dc: Dev<5>, dd: Dev<1>, dh0: Dev<4>,
    workspace: &mut dyn FnMut(usize) -> *mut c_void, stream: MambaStream,
) {
    let [bb, n, l, h, p] = x.dims;
    let r = b.dims[4];
    for (t, w) in [(&x, "x"), (&b, "B"), (&c, "C"), (&dy, "dy")] {
        t.unit_inner(w);
        t.mergeable(1, w);
    }
    dt.mergeable(2, "dt");
    for (t, w) in [(&dx, "dx"), (&db, "dB"), (&dc, "dC")] {
        t.contiguous(w);
    }
    ddt_blh.contiguous("ddt");
    let args = MambaSsd2BwdArgs {
        batch: bb as i32, seqlen: (n * l) as i32, nheads: h as i32, headdim: p as i32,
        ngroups: h as i32, dstate: r as i32,
        x: x.ptr as *const f32, x_sb: x.s(0), x_sl: x.s(2), x_sh: x.s(3),
        dt: dt.ptr as *const f32, dt_sb: dt.s(0), dt_sl: dt.s(3), dt_sh: dt.s(1),
        A: a.ptr as *const f32,
        B: b.ptr as *const f32, B_sb: b.s(0), B_sl: b.s(2), B_sg: b.s(3),
        C: c.ptr as *const f32, C_sb: c.s(0), C_sl: c.s(2), C_sg: c.s(3),
        D: d.ptr as *const f32,
        initial_state: h0.ptr as *const f32,
        dy: dy.ptr as *const f32, dy_sb: dy.s(0), dy_sl: dy.s(2), dy_sh: dy.s(3),
        d_final_state: dhf.ptr as *const f32,
        dx: dx.ptr as *mut f32, ddt: ddt_blh.ptr as *mut f32, dA: da.ptr as *mut f32,
        dB: db.ptr as *mut f32, dC: dc.ptr as *mut f32, dD: dd.ptr as *mut f32,
        d_initial_state: dh0.ptr as *mut f32,
    };
    // SAFETY: as in ssd2_forward.
    let bytes = unsafe { mamba_ssd2_bwd_workspace_size(&args) };
    let ws = if bytes > 0 { workspace(bytes) } else { core::ptr::null_mut() };
    check(unsafe { mamba_ssd2_bwd(&args, ws, bytes, stream) }, "mamba_ssd2_bwd");
}

/// `Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated`: v [b, n, l, m, h, p],
/// da / gamma / scale [b, n, l, h], B / C [b, n, l, m, h, r], initial state
/// [b, h, p, r] -> y [b, n, l, m, h, p], final state [b, h, p, r].
/// `siso_specialization` is the reference's performance switch: the library
/// handles every MIMO rank with one kernel, so it has no argument here.
#[allow(clippy::too_many_arguments)]
pub fn ssd3_single_forward(
    v: Dev<6>, da: Dev<4>, b: Dev<6>, c: Dev<6>, gamma: Dev<4>, scale: Dev<4>, h0: Dev<4>, y: Dev<6>,
    hf: Dev<4>, io_dtype: c_int, workspace: &mut dyn FnMut(usize) -> *mut c_void, stream: MambaStream,
) {
    let [bb, n, l, m, h, p] = v.dims;
    let r = b.dims[5];
    for (t, w) in [(&v, "v"), (&b, "B"), (&c, "C"), (&y, "y")] {
        t.unit_inner(w);
        t.mergeable(1, w);
    }
    for (t, w) in [(&da, "da"), (&gamma, "gamma"), (&scale, "scale")] {
        t.unit_inner(w);
        t.mergeable(1, w);
    }
    h0.contiguous("initial_state");
    hf.contiguous("final_state");
    let args = MambaSsd3Args {
        batch: bb as i32, seqlen: (n * l) as i32, mimo: m as i32, nheads: h as i32, headdim: p as i32,
        ngroups: h as i32, dstate: r as i32, chunk_len: l as i32, io_dtype,
        v: v.ptr, v_sb: v.s(0), v_sl: v.s(2), v_sm: v.s(3), v_sh: v.s(4),
        da: da.ptr as *const f32, da_sb: da.s(0), da_sl: da.s(2), da_sh: da.s(3),
        gamma: gamma.ptr as *const f32, gamma_sb: gamma.s(0), gamma_sl: gamma.s(2), gamma_sh: gamma.s(3),
        scale: scale.ptr as *const f32, scale_sb: scale.s(0), scale_sl: scale.s(2), scale_sh: scale.s(3),
        B: b.ptr, B_sb: b.s(0), B_sl: b.s(2), B_sm: b.s(3), B_sg: b.s(4),
        C: c.ptr, C_sb: c.s(0), C_sl: c.s(2), C_sm: c.s(3), C_sg: c.s(4),
        initial_state: h0.ptr as *const f32,
        y: y.ptr, y_sb: y.s(0), y_sl: y.s(2), y_sm: y.s(3), y_sh: y.s(4),
        final_state: hf.ptr as *mut f32,
    };
    // SAFETY: as in ssd2_forward.
    let bytes = unsafe { mamba_ssd3_workspace_size(&args) };
    let ws = if bytes > 0 { workspace(bytes) } else { core::ptr::null_mut() };
    check(unsafe { mamba_ssd3_fwd(&args, ws, bytes, stream) }, "mamba_ssd3_fwd");
}

/// `Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated`: the single seam
/// without gamma / scale (unit coefficients).
#[allow(clippy::too_many_arguments)]
pub fn ssd3_double_forward(
    v: Dev<6>, da: Dev<4>, b: Dev<6>, c: Dev<6>, h0: Dev<4>, y: Dev<6>, hf: Dev<4>, io_dtype: c_int,
    workspace: &mut dyn FnMut(usize) -> *mut c_void, stream: MambaStream,
) {
    let [bb, n, l, m, h, p] = v.dims;
    let r = b.dims[5];
    for (t, w) in [(&v, "v"), (&b, "B"), (&c, "C"), (&y, "y")] {
        t.unit_inner(w);
        t.mergeable(1, w);
    }
    da.mergeable(1, "da");
    h0.contiguous("initial_state");
    hf.contiguous("final_state");
    let args = MambaSsd3DoubleArgs {
        batch: bb as i32, seqlen: (n * l) as i32, mimo: m as i32, nheads: h as i32, headdim: p as i32,
        ngroups: h as i32, dstate: r as i32, chunk_len: l as i32, io_dtype,
        v: v.ptr, v_sb: v.s(0), v_sl: v.s(2), v_sm: v.s(3), v_sh: v.s(4),
        da: da.ptr as *const f32, da_sb: da.s(0), da_sl: da.s(2), da_sh: da.s(3),
        B: b.ptr, B_sb: b.s(0), B_sl: b.s(2), B_sm: b.s(3), B_sg: b.s(4),
        C: c.ptr, C_sb: c.s(0), C_sl: c.s(2), C_sm: c.s(3), C_sg: c.s(4),
        initial_state: h0.ptr as *const f32,
        y: y.ptr, y_sb: y.s(0), y_sl: y.s(2), y_sm: y.s(3), y_sh: y.s(4),
        final_state: hf.ptr as *mut f32,
    };
    // SAFETY: as in ssd2_forward.
    let bytes = unsafe { mamba_ssd3_double_workspace_size(&args) };
    let ws = if bytes > 0 { workspace(bytes) } else { core::ptr::null_mut() };
    check(unsafe { mamba_ssd3_double_fwd(&args, ws, bytes, stream) }, "mamba_ssd3_double_fwd");
}

/// The gradients of the Mamba-3 seams (single: `single_ssd/ssd/serial_recalculated/
/// backward.rs:27-299`; double, with `gamma = scale = None`: `double_ssd/ssd/
/// serial_recalculated/backward.rs:27-275`), f32, all outputs contiguous in
/// the seam's layouts: dv [b, n, l, m, h, p], dda / dgamma / dscale
/// [b, n, l, h], dB / dC [b, n, l, m, h, r], d(initial state) [b, h, p, r].
#[allow(clippy::too_many_arguments)]
pub fn ssd3_backward(
    v: Dev<6>, da: Dev<4>, b: Dev<6>, c: Dev<6>, gamma: Option<Dev<4>>, scale: Option<Dev<4>>, h0: Dev<4>,
    dy: Dev<6>, dhf: Dev<4>, dv: Dev<6>, dda: Dev<4>, dgamma: Option<Dev<4>>, dscale: Option<Dev<4>>,
    db: Dev<6>, dc: Dev<6>, dh0: Dev<4>, workspace: &mut dyn FnMut(usize) -> *mut c_void, stream: MambaStream,
) {
    let [bb, n, l, m, h, p] = v.dims;
    let r = b.dims[5];
    for (t, w) in [(&v, "v"), (&b, "B"), (&c, "C"), (&dy, "dy")] {
        t.unit_inner(w);
        t.mergeable(1, w);
    }
    for (t, w) in [(&dv, "dv"), (&db, "dB"), (&dc, "dC")] {
        t.contiguous(w);
    }
    dda.contiguous("dda");
    let g = gamma.unwrap_or(Dev { ptr: core::ptr::null_mut(), dims: [0; 4], strides: [0; 4] });
    let s = scale.unwrap_or(Dev { ptr: core::ptr::null_mut(), dims: [0; 4], strides: [0; 4] });
    let args = MambaSsd3BwdArgs {
        batch: bb as i32, seqlen: (n * l) as i32, mimo: m as i32, nheads: h as i32, headdim: p as i32,
        ngroups: h as i32, dstate: r as i32,
        v: v.ptr as *const f32, v_sb: v.s(0), v_sl: v.s(2), v_sm: v.s(3), v_sh: v.s(4),
        da: da.ptr as *const f32, da_sb: da.s(0), da_sl: da.s(2), da_sh: da.s(3),
        gamma: g.ptr as *const f32, gamma_sb: g.s(0), gamma_sl: g.s(2), gamma_sh: g.s(3),
        scale: s.ptr as *const f32, scale_sb: s.s(0), scale_sl: s.s(2), scale_sh: s.s(3),
        B: b.ptr as *const f32, B_sb: b.s(0), B_sl: b.s(2), B_sm: b.s(3), B_sg: b.s(4),
        C: c.ptr as *const f32, C_sb: c.s(0), C_sl: c.s(2), C_sm: c.s(3), C_sg: c.s(4),
        initial_state: h0.ptr as *const f32,
        dy: dy.ptr as *const f32, dy_sb: dy.s(0), dy_sl: dy.s(2), dy_sm: dy.s(3), dy_sh: dy.s(4),
        d_final_state: dhf.ptr as *const f32,
        dv: dv.ptr as *mut f32, dda: dda.ptr as *mut f32,
        dgamma: dgamma.map_or(core::ptr::null_mut(), |t| t.ptr as *mut f32),
        dscale: dscale.map_or(core::ptr::null_mut(), |t| t.ptr as *mut f32),
        dB: db.ptr as *mut f32, dC: dc.ptr as *mut f32, d_initial_state: dh0.ptr as *mut f32,
    };
    // SAFETY: as in ssd2_forward.
    let bytes = unsafe { mamba_ssd3_bwd_workspace_size(&args) };
    let ws = if bytes > 0 { workspace(bytes) } else { core::ptr::null_mut() };
    check(unsafe { mamba_ssd3_bwd(&args, ws, bytes, stream) }, "mamba_ssd3_bwd");
}

#[cfg(test)]
mod tests {
    use super::*;

    fn contiguous<const R: usize>(dims: [usize; R]) -> Dev<R> {
        let mut strides = [0isize; R];
        let mut s = 1isize;
        for i in (0..R).rev() {
            strides[i] = s;
            s *= dims[i] as isize;
        }
        Dev { ptr: core::ptr::null_mut(), dims, strides }
    }

    #[test]
    fn chunked_axes_merge() {
        let x = contiguous([2, 4, 64, 8, 16]);
        x.mergeable(1, "x");
        let dt = contiguous([2, 8, 4, 64]);
        dt.mergeable(2, "dt");
        assert_eq!(dt.s(3), 1);
        assert_eq!(dt.s(1), 4 * 64);
    }

    #[test]
    #[should_panic]
    fn unmergeable_axes_are_refused() {
        let mut x = contiguous([2, 4, 64, 8, 16]);
        x.strides[1] += 1;
        x.mergeable(1, "x");
    }
}
