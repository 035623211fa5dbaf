// Generated from include/mamba_hip.h by gen_ffi.py: do not edit by hand.
// One #[repr(C)] struct per argument struct (same fields, same order) and one
// extern "C" declaration per entry point.
#![allow(non_snake_case, non_camel_case_types, clippy::upper_case_acronyms)]

use core::ffi::{c_char, c_int, c_void};

/// hipStream_t (a pointer); null is the default stream.
pub type MambaStream = *mut c_void;

pub const MAMBA_OK: c_int = 0;
pub const MAMBA_ERR_INVALID_ARG: c_int = 1;
pub const MAMBA_ERR_UNSUPPORTED: c_int = 2;
pub const MAMBA_ERR_WORKSPACE: c_int = 3;
pub const MAMBA_ERR_HIP: c_int = 4;
pub const MAMBA_F32: c_int = 0;
pub const MAMBA_BF16: c_int = 1;
pub const MAMBA2_STACK_NOALLOC_SCRATCH_BYTES: usize = 48 << 20;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaSsd2Args {
    pub batch: i32,
    pub seqlen: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub chunk_len: i32,
    pub io_dtype: i32,
    pub x: *const c_void,
    pub x_sb: i64,
    pub x_sl: i64,
    pub x_sh: i64,
    pub dt: *const f32,
    pub dt_sb: i64,
    pub dt_sl: i64,
    pub dt_sh: i64,
    pub A: *const f32,
    pub B: *const c_void,
    pub B_sb: i64,
    pub B_sl: i64,
    pub B_sg: i64,
    pub C: *const c_void,
    pub C_sb: i64,
    pub C_sl: i64,
    pub C_sg: i64,
    pub D: *const f32,
    pub initial_state: *const f32,
    pub init_state_hpr: *const f32,
    pub y: *mut c_void,
    pub y_sb: i64,
    pub y_sl: i64,
    pub y_sh: i64,
    pub final_state: *mut f32,
}

impl Default for MambaSsd2Args {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaSsd2BwdArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub x: *const f32,
    pub x_sb: i64,
    pub x_sl: i64,
    pub x_sh: i64,
    pub dt: *const f32,
    pub dt_sb: i64,
    pub dt_sl: i64,
    pub dt_sh: i64,
    pub A: *const f32,
    pub B: *const f32,
    pub B_sb: i64,
    pub B_sl: i64,
    pub B_sg: i64,
    pub C: *const f32,
    pub C_sb: i64,
    pub C_sl: i64,
    pub C_sg: i64,
    pub D: *const f32,
    pub initial_state: *const f32,
    pub dy: *const f32,
    pub dy_sb: i64,
    pub dy_sl: i64,
    pub dy_sh: i64,
    pub d_final_state: *const f32,
    pub dx: *mut f32,
    pub ddt: *mut f32,
    pub dA: *mut f32,
    pub dB: *mut f32,
    pub dC: *mut f32,
    pub dD: *mut f32,
    pub d_initial_state: *mut f32,
}

impl Default for MambaSsd2BwdArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaSsd3Args {
    pub batch: i32,
    pub seqlen: i32,
    pub mimo: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub chunk_len: i32,
    pub io_dtype: i32,
    pub v: *const c_void,
    pub v_sb: i64,
    pub v_sl: i64,
    pub v_sm: i64,
    pub v_sh: i64,
    pub da: *const f32,
    pub da_sb: i64,
    pub da_sl: i64,
    pub da_sh: i64,
    pub gamma: *const f32,
    pub gamma_sb: i64,
    pub gamma_sl: i64,
    pub gamma_sh: i64,
    pub scale: *const f32,
    pub scale_sb: i64,
    pub scale_sl: i64,
    pub scale_sh: i64,
    pub B: *const c_void,
    pub B_sb: i64,
    pub B_sl: i64,
    pub B_sm: i64,
    pub B_sg: i64,
    pub C: *const c_void,
    pub C_sb: i64,
    pub C_sl: i64,
    pub C_sm: i64,
    pub C_sg: i64,
    pub initial_state: *const f32,
    pub y: *mut c_void,
    pub y_sb: i64,
    pub y_sl: i64,
    pub y_sm: i64,
    pub y_sh: i64,
    pub final_state: *mut f32,
}

impl Default for MambaSsd3Args {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaSsd3DoubleArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub mimo: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub chunk_len: i32,
    pub io_dtype: i32,
    pub v: *const c_void,
    pub v_sb: i64,
    pub v_sl: i64,
    pub v_sm: i64,
    pub v_sh: i64,
    pub da: *const f32,
    pub da_sb: i64,
    pub da_sl: i64,
    pub da_sh: i64,
    pub B: *const c_void,
    pub B_sb: i64,
    pub B_sl: i64,
    pub B_sm: i64,
    pub B_sg: i64,
    pub C: *const c_void,
    pub C_sb: i64,
    pub C_sl: i64,
    pub C_sm: i64,
    pub C_sg: i64,
    pub initial_state: *const f32,
    pub y: *mut c_void,
    pub y_sb: i64,
    pub y_sl: i64,
    pub y_sm: i64,
    pub y_sh: i64,
    pub final_state: *mut f32,
}

impl Default for MambaSsd3DoubleArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaSsd3BwdArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub mimo: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub v: *const f32,
    pub v_sb: i64,
    pub v_sl: i64,
    pub v_sm: i64,
    pub v_sh: i64,
    pub da: *const f32,
    pub da_sb: i64,
    pub da_sl: i64,
    pub da_sh: i64,
    pub gamma: *const f32,
    pub gamma_sb: i64,
    pub gamma_sl: i64,
    pub gamma_sh: i64,
    pub scale: *const f32,
    pub scale_sb: i64,
    pub scale_sl: i64,
    pub scale_sh: i64,
    pub B: *const f32,
    pub B_sb: i64,
    pub B_sl: i64,
    pub B_sm: i64,
    pub B_sg: i64,
    pub C: *const f32,
    pub C_sb: i64,
    pub C_sl: i64,
    pub C_sm: i64,
    pub C_sg: i64,
    pub initial_state: *const f32,
    pub dy: *const f32,
    pub dy_sb: i64,
    pub dy_sl: i64,
    pub dy_sm: i64,
    pub dy_sh: i64,
    pub d_final_state: *const f32,
    pub dv: *mut f32,
    pub dda: *mut f32,
    pub dgamma: *mut f32,
    pub dscale: *mut f32,
    pub dB: *mut f32,
    pub dC: *mut f32,
    pub d_initial_state: *mut f32,
}

impl Default for MambaSsd3BwdArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba1ScanArgs {
    pub batch: i32,
    pub dim: i32,
    pub seqlen: i32,
    pub dstate: i32,
    pub u: *const f32,
    pub u_sb: i64,
    pub u_sd: i64,
    pub u_sl: i64,
    pub delta: *const f32,
    pub delta_sb: i64,
    pub delta_sd: i64,
    pub delta_sl: i64,
    pub A: *const f32,
    pub A_sd: i64,
    pub A_sn: i64,
    pub B: *const f32,
    pub B_sb: i64,
    pub B_sn: i64,
    pub B_sl: i64,
    pub C: *const f32,
    pub C_sb: i64,
    pub C_sn: i64,
    pub C_sl: i64,
    pub D: *const f32,
    pub z: *const f32,
    pub z_sb: i64,
    pub z_sd: i64,
    pub z_sl: i64,
    pub delta_bias: *const f32,
    pub delta_softplus: i32,
    pub initial_state: *const f32,
    pub y: *mut f32,
    pub y_sb: i64,
    pub y_sd: i64,
    pub y_sl: i64,
    pub final_state: *mut f32,
}

impl Default for Mamba1ScanArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba1StepArgs {
    pub batch: i32,
    pub dim: i32,
    pub dstate: i32,
    pub u: *const f32,
    pub u_sb: i64,
    pub delta: *const f32,
    pub delta_sb: i64,
    pub A: *const f32,
    pub A_sd: i64,
    pub A_sn: i64,
    pub B: *const f32,
    pub B_sb: i64,
    pub B_sn: i64,
    pub C: *const f32,
    pub C_sb: i64,
    pub C_sn: i64,
    pub D: *const f32,
    pub z: *const f32,
    pub z_sb: i64,
    pub delta_bias: *const f32,
    pub delta_softplus: i32,
    pub state: *mut f32,
    pub y: *mut f32,
    pub y_sb: i64,
}

impl Default for Mamba1StepArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaConv1dStepArgs {
    pub batch: i32,
    pub channels: i32,
    pub kernel: i32,
    pub x_dtype: i32,
    pub out_dtype: i32,
    pub x: *const c_void,
    pub x_sb: i64,
    pub state: *mut f32,
    pub w: *const f32,
    pub bias: *const f32,
    pub silu: i32,
    pub out: *mut c_void,
    pub out_sb: i64,
}

impl Default for MambaConv1dStepArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba3StepArgs {
    pub batch: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub mimo: i32,
    pub rope_dim: i32,
    pub proj_dtype: i32,
    pub out_dtype: i32,
    pub proj: *const c_void,
    pub proj_sb: i64,
    pub ssm_state: *mut f32,
    pub k_state: *mut f32,
    pub v_state: *mut f32,
    pub angle: *mut f32,
    pub dt_bias: *const f32,
    pub a_floor: f32,
    pub dt_min: f32,
    pub dt_max: f32,
    pub rotation_range: f32,
    pub b_norm_w: *const f32,
    pub c_norm_w: *const f32,
    pub b_bias: *const f32,
    pub c_bias: *const f32,
    pub mimo_x: *const f32,
    pub mimo_z: *const f32,
    pub mimo_o: *const f32,
    pub D: *const f32,
    pub out_norm_w: *const f32,
    pub out: *mut c_void,
    pub out_sb: i64,
}

impl Default for Mamba3StepArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba3PrepArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub mimo: i32,
    pub rope_dim: i32,
    pub proj_dtype: i32,
    pub io_dtype: i32,
    pub proj: *const c_void,
    pub proj_sb: i64,
    pub proj_sl: i64,
    pub ssm_state: *const f32,
    pub k_state: *mut f32,
    pub v_state: *mut f32,
    pub angle: *const f32,
    pub angle_out: *mut f32,
    pub dt_bias: *const f32,
    pub a_floor: f32,
    pub dt_min: f32,
    pub dt_max: f32,
    pub rotation_range: f32,
    pub b_norm_w: *const f32,
    pub c_norm_w: *const f32,
    pub b_bias: *const f32,
    pub c_bias: *const f32,
    pub mimo_x: *const f32,
    pub v: *mut c_void,
    pub B: *mut c_void,
    pub C: *mut c_void,
    pub da: *mut f32,
    pub gamma: *mut f32,
    pub scale: *mut f32,
    pub initial_state: *mut f32,
}

impl Default for Mamba3PrepArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba3FinishArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub mimo: i32,
    pub io_dtype: i32,
    pub z_dtype: i32,
    pub out_dtype: i32,
    pub y_ssd: *const c_void,
    pub v: *const c_void,
    pub z: *const c_void,
    pub z_sb: i64,
    pub z_sl: i64,
    pub D: *const f32,
    pub mimo_z: *const f32,
    pub mimo_o: *const f32,
    pub out_norm_w: *const f32,
    pub out: *mut c_void,
    pub out_sb: i64,
    pub out_sl: i64,
    pub y_ranks: i32,
}

impl Default for Mamba3FinishArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba3FusedArgs {
    pub prep: Mamba3PrepArgs,
    pub D: *const f32,
    pub y: *mut c_void,
    pub final_state: *mut f32,
}

impl Default for Mamba3FusedArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba3DoubleInputsArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub mimo: i32,
    pub proj_dtype: i32,
    pub io_dtype: i32,
    pub proj: *const c_void,
    pub proj_sb: i64,
    pub proj_sl: i64,
    pub dt_bias: *const f32,
    pub a_floor: f32,
    pub dt_min: f32,
    pub dt_max: f32,
    pub v: *const c_void,
    pub B: *const c_void,
    pub C: *const c_void,
    pub x_prev: *const f32,
    pub k_prev: *const f32,
    pub mimo_x: *const f32,
    pub v2: *mut c_void,
    pub B2: *mut c_void,
    pub C2: *mut c_void,
}

impl Default for Mamba3DoubleInputsArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba2StepArgs {
    pub batch: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub conv_kernel: i32,
    pub zxbcdt_dtype: i32,
    pub out_dtype: i32,
    pub norm_before_gate: i32,
    pub zxbcdt: *const c_void,
    pub zxbcdt_sb: i64,
    pub conv_state: *mut f32,
    pub conv_w: *const f32,
    pub conv_b: *const f32,
    pub dt_bias: *const f32,
    pub A: *const f32,
    pub D: *const f32,
    pub dt_min: f32,
    pub dt_max: f32,
    pub norm_w: *const f32,
    pub ssm_state: *mut f32,
    pub out: *mut c_void,
    pub out_sb: i64,
}

impl Default for Mamba2StepArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaLinearArgs {
    pub rows: i32,
    pub d_in: i32,
    pub d_out: i32,
    pub x_dtype: i32,
    pub y_dtype: i32,
    pub x: *const c_void,
    pub x_ld: i64,
    pub packed_w: *const c_void,
    pub bias: *const f32,
    pub y: *mut c_void,
    pub y_ld: i64,
}

impl Default for MambaLinearArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba2LayerArgs {
    pub batch: i32,
    pub d_model: i32,
    pub nheads: i32,
    pub headdim: i32,
    pub ngroups: i32,
    pub dstate: i32,
    pub conv_kernel: i32,
    pub norm_before_gate: i32,
    pub zxbcdt_dtype: i32,
    pub x: *mut f32,
    pub x_sb: i64,
    pub pre_norm_w: *const f32,
    pub in_proj: *const c_void,
    pub in_proj_b: *const f32,
    pub out_proj: *const c_void,
    pub out_proj_b: *const f32,
    pub conv_state: *mut f32,
    pub conv_w: *const f32,
    pub conv_b: *const f32,
    pub dt_bias: *const f32,
    pub A: *const f32,
    pub D: *const f32,
    pub dt_min: f32,
    pub dt_max: f32,
    pub norm_w: *const f32,
    pub ssm_state: *mut f32,
    pub concurrent: i32,
}

impl Default for Mamba2LayerArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MambaRmsnormArgs {
    pub rows: i32,
    pub cols: i32,
    pub add_dtype: i32,
    pub out_dtype: i32,
    pub x: *mut f32,
    pub x_sr: i64,
    pub add: *const c_void,
    pub add_sr: i64,
    pub weight: *const f32,
    pub out: *mut c_void,
    pub out_sr: i64,
}

impl Default for MambaRmsnormArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba2ConvArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub channels: i32,
    pub kernel: i32,
    pub nheads: i32,
    pub in_dtype: i32,
    pub out_dtype: i32,
    pub proj: *const c_void,
    pub proj_sb: i64,
    pub proj_sl: i64,
    pub xbc_offset: i32,
    pub dt_offset: i32,
    pub conv_w: *const f32,
    pub conv_b: *const f32,
    pub conv_state: *mut f32,
    pub dt_bias: *const f32,
    pub dt_min: f32,
    pub dt_max: f32,
    pub xbc: *mut c_void,
    pub xbc_sb: i64,
    pub xbc_sl: i64,
    pub dt: *mut f32,
}

impl Default for Mamba2ConvArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct Mamba2GatedNormArgs {
    pub batch: i32,
    pub seqlen: i32,
    pub width: i32,
    pub norm_before_gate: i32,
    pub y_dtype: i32,
    pub z_dtype: i32,
    pub out_dtype: i32,
    pub eps: f32,
    pub y: *const c_void,
    pub y_sb: i64,
    pub y_sl: i64,
    pub z: *const c_void,
    pub z_sb: i64,
    pub z_sl: i64,
    pub gamma: *const f32,
    pub out: *mut c_void,
    pub out_sb: i64,
    pub out_sl: i64,
}

impl Default for Mamba2GatedNormArgs {
    /// Every size 0, every pointer null, every stride 0.
    fn default() -> Self {
        // SAFETY: all fields are integers, floats or raw pointers, for which zero is valid.
        unsafe { core::mem::zeroed() }
    }
}

extern "C" {
    pub fn mamba_last_error() -> *const c_char;
    pub fn mamba_version() -> *const c_char;
    pub fn mamba_ssd2_workspace_size(args: *const MambaSsd2Args) -> usize;
    pub fn mamba_ssd2_fast_path(args: *const MambaSsd2Args) -> c_int;
    pub fn mamba_ssd2_fwd(args: *const MambaSsd2Args, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd2_fwd_generic(args: *const MambaSsd2Args, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd2_fwd_timed(args: *const MambaSsd2Args, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba_ssd2_bwd_workspace_size(args: *const MambaSsd2BwdArgs) -> usize;
    pub fn mamba_ssd2_bwd(args: *const MambaSsd2BwdArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd2_bwd_timed(args: *const MambaSsd2BwdArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba_ssd3_workspace_size(args: *const MambaSsd3Args) -> usize;
    pub fn mamba_ssd3_fast_path(args: *const MambaSsd3Args) -> c_int;
    pub fn mamba_ssd3_fwd(args: *const MambaSsd3Args, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd3_fwd_generic(args: *const MambaSsd3Args, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd3_fwd_timed(args: *const MambaSsd3Args, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba_ssd3_double_workspace_size(args: *const MambaSsd3DoubleArgs) -> usize;
    pub fn mamba_ssd3_double_fast_path(args: *const MambaSsd3DoubleArgs) -> c_int;
    pub fn mamba_ssd3_double_fwd(args: *const MambaSsd3DoubleArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd3_double_fwd_generic(args: *const MambaSsd3DoubleArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd3_bwd_workspace_size(args: *const MambaSsd3BwdArgs) -> usize;
    pub fn mamba_ssd3_bwd(args: *const MambaSsd3BwdArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba_ssd3_bwd_timed(args: *const MambaSsd3BwdArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba1_scan_fwd(args: *const Mamba1ScanArgs, stream: MambaStream) -> c_int;
    pub fn mamba1_scan_fwd_timed(args: *const Mamba1ScanArgs, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba1_scan_step(args: *const Mamba1StepArgs, stream: MambaStream) -> c_int;
    pub fn mamba1_scan_step_timed(args: *const Mamba1StepArgs, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba_conv1d_step(args: *const MambaConv1dStepArgs, stream: MambaStream) -> c_int;
    pub fn mamba3_step_ssm(args: *const Mamba3StepArgs, stream: MambaStream) -> c_int;
    pub fn mamba3_step_ssm_timed(args: *const Mamba3StepArgs, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba3_prep_fast_path(args: *const Mamba3PrepArgs) -> c_int;
    pub fn mamba3_prep_workspace_size(args: *const Mamba3PrepArgs) -> usize;
    pub fn mamba3_prep_fwd(args: *const Mamba3PrepArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba3_finish_fwd(args: *const Mamba3FinishArgs, stream: MambaStream) -> c_int;
    pub fn mamba3_ssd_fused_supported(args: *const Mamba3FusedArgs) -> c_int;
    pub fn mamba3_ssd_fused_fwd(args: *const Mamba3FusedArgs, stream: MambaStream) -> c_int;
    pub fn mamba3_ssd_fused_fwd_timed(args: *const Mamba3FusedArgs, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba3_double_inputs(args: *const Mamba3DoubleInputsArgs, stream: MambaStream) -> c_int;
    pub fn mamba2_step_workspace_size(args: *const Mamba2StepArgs) -> usize;
    pub fn mamba2_step_ssm(args: *const Mamba2StepArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba2_step_ssm_timed(args: *const Mamba2StepArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba_linear_packed_size(d_in: i32, d_out: i32) -> usize;
    pub fn mamba_linear_pack(weight: *const c_void, d_in: i32, d_out: i32, ld: i64, dtype: i32, packed: *mut c_void, stream: MambaStream) -> c_int;
    pub fn mamba_linear_workspace_size(args: *const MambaLinearArgs) -> usize;
    pub fn mamba_linear_fwd(args: *const MambaLinearArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba2_layer_workspace_size(args: *const Mamba2LayerArgs) -> usize;
    pub fn mamba2_layer_step(args: *const Mamba2LayerArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba2_layer_step_timed(args: *const Mamba2LayerArgs, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *mut c_void, event_stop: *mut c_void) -> c_int;
    pub fn mamba2_stack_step(layers: *const Mamba2LayerArgs, n_layers: i32, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream) -> c_int;
    pub fn mamba2_stack_step_timed(layers: *const Mamba2LayerArgs, n_layers: i32, workspace: *mut c_void, workspace_bytes: usize, stream: MambaStream, event_start: *const *mut c_void, event_stop: *const *mut c_void) -> c_int;
    pub fn mamba2_stack_step_noalloc(layers: *const Mamba2LayerArgs, n_layers: i32, stream: MambaStream) -> c_int;
    pub fn mamba_rmsnorm(args: *const MambaRmsnormArgs, stream: MambaStream) -> c_int;
    pub fn mamba2_conv_fwd(args: *const Mamba2ConvArgs, stream: MambaStream) -> c_int;
    pub fn mamba2_gated_rmsnorm(args: *const Mamba2GatedNormArgs, stream: MambaStream) -> c_int;
}
