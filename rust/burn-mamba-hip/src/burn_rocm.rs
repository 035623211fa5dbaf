//! The ROCm arms of burn-mamba's SSD backend-extension traits, as functions on
//! Burn's HIP tensors (`burn_cubecl::tensor::CubeTensor<cubecl_hip::HipRuntime>`):
//! each allocates its outputs on the tensors' device and calls `seams` on the
//! stream CubeCL submits to, so the call is ordered with Burn's own kernels.
//! burn-mamba's trait impls for `CubeBackend<HipRuntime>` (the patch under
//! `patches/`) delegate to these.
//!
//! Three functions touch Burn / CubeCL internals at the revision burn-mamba
//! pins (git 1893b608, its Cargo.lock): `dev` (a handle's device pointer and
//! the tensor's strides), `empty` (a device allocation of a shape) and
//! `stream_of` (CubeCL's HIP stream of a device).  Everything else goes
//! through `seams`, which depends only on the C ABI.

use core::ffi::c_void;
use std::collections::HashMap;
use std::sync::Mutex;

use burn_cubecl::tensor::CubeTensor;
use burn_cubecl::CubeRuntime;
use burn_tensor::{DType, Shape};
use cubecl_hip::HipRuntime;

use crate::ffi::{MambaStream, MAMBA_BF16, MAMBA_F32};
use crate::seams::{self, Dev};

type T = CubeTensor<HipRuntime>;

/// The tensor's device pointer (its handle's binding resource, plus the
/// handle's offset) with its shape and element strides.
fn dev<const R: usize>(t: &T) -> Dev<R> {
    let resource = t.client.get_resource(t.handle.clone().binding());
    let ptr = resource.resource().ptr as *mut c_void;
    let dims: [usize; R] = t.shape.dims::<R>();
    let mut strides = [0isize; R];
    for (s, v) in strides.iter_mut().zip(t.strides.iter()) {
        *s = *v as isize;
    }
    Dev { ptr, dims, strides }
}

/// An uninitialised contiguous tensor of `dims` on `like`'s device.
fn empty(like: &T, dims: &[usize], dtype: DType) -> T {
    let shape = Shape::from(dims.to_vec());
    burn_cubecl::ops::numeric::empty_device_dtype::<HipRuntime>(like.client.clone(), like.device.clone(), shape, dtype)
}

/// The HIP stream CubeCL submits to for `t`'s device.  The library's calls
/// go on it, so they are ordered with CubeCL's kernels without a host sync.
fn stream_of(t: &T) -> MambaStream {
    t.client.stream_handle() as MambaStream
}

fn io_dtype(t: &T) -> i32 {
    match t.dtype {
        DType::BF16 => MAMBA_BF16,
        DType::F32 => MAMBA_F32,
        other => panic!("burn-mamba-hip: SSD inputs must be f32 or bf16, got {other:?}"),
    }
}

/// A per-device workspace that grows to the largest request and is kept
/// (the library never allocates).
static WORKSPACES: Mutex<Option<HashMap<usize, T>>> = Mutex::new(None);

fn workspace(like: &T) -> impl FnMut(usize) -> *mut c_void + '_ {
    move |bytes| {
        let mut all = WORKSPACES.lock().unwrap();
        let map = all.get_or_insert_with(HashMap::new);
        let key = like.device.index();
        let need = bytes.div_ceil(4);
        let fits = map.get(&key).map_or(false, |w| w.shape.num_elements() >= need);
        if !fits {
            map.insert(key, empty(like, &[need], DType::F32));
        }
        dev::<1>(&map[&key]).ptr
    }
}

/// `Mamba2BackendExt::ssd_serial_recalculated` on ROCm.
pub fn ssd2_forward(x: T, dt: T, b: T, c: T, d: T, h0: T, a: T) -> (T, T) {
    let [bb, n, l, h, p] = x.shape.dims::<5>();
    let r = b.shape.dims::<5>()[4];
    let y = empty(&x, &[bb, n, l, h, p], x.dtype);
    let hf = empty(&x, &[bb, h, p, r], DType::F32);
    seams::ssd2_forward(
        dev(&x), dev(&dt), dev(&b), dev(&c), dev(&d), dev(&h0), dev(&a), dev(&y), dev(&hf), io_dtype(&x),
        &mut workspace(&x), stream_of(&x),
    );
    (y, hf)
}

/// The gradients of `ssd2_forward` for the Autodiff arm's backward node:
/// (dx, ddt, dB, dC, dD, d(initial state), dA) in the seam's layouts.
#[allow(clippy::too_many_arguments)]
pub fn ssd2_backward(x: T, dt: T, b: T, c: T, d: T, h0: T, a: T, dy: T, dhf: T) -> [T; 7] {
    let [bb, n, l, h, p] = x.shape.dims::<5>();
    let r = b.shape.dims::<5>()[4];
    let f = DType::F32;
    let dx = empty(&x, &[bb, n, l, h, p], f);
    let ddt_blh = empty(&x, &[bb, n * l, h], f);
    let da = empty(&x, &[h], f);
    let db = empty(&x, &[bb, n, l, h, r], f);
    let dc = empty(&x, &[bb, n, l, h, r], f);
    let dd = empty(&x, &[h], f);
    let dh0 = empty(&x, &[bb, h, p, r], f);
    seams::ssd2_backward(
        dev(&x), dev(&dt), dev(&b), dev(&c), dev(&d), dev(&h0), dev(&a), dev(&dy), dev(&dhf), dev(&dx),
        dev(&ddt_blh), dev(&da), dev(&db), dev(&dc), dev(&dd), dev(&dh0), &mut workspace(&x), stream_of(&x),
    );
    // the seam's dt is [b, h, n, l]: the library's position-major gradient, permuted
    let ddt = burn_cubecl::ops::permute(ddt_blh, &[0, 2, 1]);
    let ddt = burn_cubecl::ops::reshape(burn_cubecl::kernel::into_contiguous(ddt), Shape::from([bb, h, n, l]));
    [dx, ddt, db, dc, dd, dh0, da]
}

/// `Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated` on ROCm.
#[allow(clippy::too_many_arguments)]
pub fn ssd3_single_forward(v: T, da: T, b: T, c: T, gamma: T, scale: T, h0: T) -> (T, T) {
    let [bb, n, l, m, h, p] = v.shape.dims::<6>();
    let r = b.shape.dims::<6>()[5];
    let y = empty(&v, &[bb, n, l, m, h, p], v.dtype);
    let hf = empty(&v, &[bb, h, p, r], DType::F32);
    seams::ssd3_single_forward(
        dev(&v), dev(&da), dev(&b), dev(&c), dev(&gamma), dev(&scale), dev(&h0), dev(&y), dev(&hf), io_dtype(&v),
        &mut workspace(&v), stream_of(&v),
    );
    (y, hf)
}

/// `Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated` on ROCm.
pub fn ssd3_double_forward(v: T, da: T, b: T, c: T, h0: T) -> (T, T) {
    let [bb, n, l, m, h, p] = v.shape.dims::<6>();
    let r = b.shape.dims::<6>()[5];
    let y = empty(&v, &[bb, n, l, m, h, p], v.dtype);
    let hf = empty(&v, &[bb, h, p, r], DType::F32);
    seams::ssd3_double_forward(
        dev(&v), dev(&da), dev(&b), dev(&c), dev(&h0), dev(&y), dev(&hf), io_dtype(&v), &mut workspace(&v),
        stream_of(&v),
    );
    (y, hf)
}

/// The gradients of the Mamba-3 seams for their Autodiff arms: (dv, dda, dB,
/// dC, d(initial state), dgamma, dscale); the last two are None for the
/// double seam (`gamma = scale = None`).
#[allow(clippy::too_many_arguments)]
pub fn ssd3_backward(
    v: T, da: T, b: T, c: T, gamma: Option<T>, scale: Option<T>, h0: T, dy: T, dhf: T,
) -> (T, T, T, T, T, Option<T>, Option<T>) {
    let [bb, n, l, m, h, p] = v.shape.dims::<6>();
    let r = b.shape.dims::<6>()[5];
    let f = DType::F32;
    let dv = empty(&v, &[bb, n, l, m, h, p], f);
    let dda = empty(&v, &[bb, n, l, h], f);
    let db = empty(&v, &[bb, n, l, m, h, r], f);
    let dc = empty(&v, &[bb, n, l, m, h, r], f);
    let dh0 = empty(&v, &[bb, h, p, r], f);
    let dg = gamma.as_ref().map(|_| empty(&v, &[bb, n, l, h], f));
    let ds = scale.as_ref().map(|_| empty(&v, &[bb, n, l, h], f));
    seams::ssd3_backward(
        dev(&v), dev(&da), dev(&b), dev(&c), gamma.as_ref().map(dev), scale.as_ref().map(dev), dev(&h0),
        dev(&dy), dev(&dhf), dev(&dv), dev(&dda), dg.as_ref().map(dev), ds.as_ref().map(dev), dev(&db), dev(&dc),
        dev(&dh0), &mut workspace(&v), stream_of(&v),
    );
    (dv, dda, db, dc, dh0, dg, ds)
}
