"""ctypes binding of libmamba_hip.so (include/mamba_hip.h).

The library is the product: there is no fallback.  If it is missing, loading
raises; if a call returns a non-zero status, ``MambaHipError`` is raised with
the library's own message (the reference panics via ``assert!`` in the same
situations).  Device memory and streams come from PyTorch (ROCm build) as
plain pointers.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "..", "lib", "libmamba_hip.so")

MAMBA_F32 = 0
MAMBA_BF16 = 1

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p


class MambaHipError(RuntimeError):
    pass


class Ssd2Args(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("nheads", c_i32), ("headdim", c_i32),
        ("ngroups", c_i32), ("dstate", c_i32), ("chunk_len", c_i32), ("io_dtype", c_i32),
        ("x", c_vp), ("x_sb", c_i64), ("x_sl", c_i64), ("x_sh", c_i64),
        ("dt", c_vp), ("dt_sb", c_i64), ("dt_sl", c_i64), ("dt_sh", c_i64),
        ("A", c_vp),
        ("B", c_vp), ("B_sb", c_i64), ("B_sl", c_i64), ("B_sg", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sl", c_i64), ("C_sg", c_i64),
        ("D", c_vp), ("initial_state", c_vp), ("init_state_hpr", c_vp),
        ("y", c_vp), ("y_sb", c_i64), ("y_sl", c_i64), ("y_sh", c_i64),
        ("final_state", c_vp),
    ]


class Ssd3Args(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("mimo", c_i32), ("nheads", c_i32), ("headdim", c_i32),
        ("ngroups", c_i32), ("dstate", c_i32), ("chunk_len", c_i32), ("io_dtype", c_i32),
        ("v", c_vp), ("v_sb", c_i64), ("v_sl", c_i64), ("v_sm", c_i64), ("v_sh", c_i64),
        ("da", c_vp), ("da_sb", c_i64), ("da_sl", c_i64), ("da_sh", c_i64),
        ("gamma", c_vp), ("gamma_sb", c_i64), ("gamma_sl", c_i64), ("gamma_sh", c_i64),
        ("scale", c_vp), ("scale_sb", c_i64), ("scale_sl", c_i64), ("scale_sh", c_i64),
        ("B", c_vp), ("B_sb", c_i64), ("B_sl", c_i64), ("B_sm", c_i64), ("B_sg", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sl", c_i64), ("C_sm", c_i64), ("C_sg", c_i64),
        ("initial_state", c_vp),
        ("y", c_vp), ("y_sb", c_i64), ("y_sl", c_i64), ("y_sm", c_i64), ("y_sh", c_i64),
        ("final_state", c_vp),
    ]


class Ssd3DoubleArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("mimo", c_i32), ("nheads", c_i32), ("headdim", c_i32),
        ("ngroups", c_i32), ("dstate", c_i32), ("chunk_len", c_i32), ("io_dtype", c_i32),
        ("v", c_vp), ("v_sb", c_i64), ("v_sl", c_i64), ("v_sm", c_i64), ("v_sh", c_i64),
        ("da", c_vp), ("da_sb", c_i64), ("da_sl", c_i64), ("da_sh", c_i64),
        ("B", c_vp), ("B_sb", c_i64), ("B_sl", c_i64), ("B_sm", c_i64), ("B_sg", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sl", c_i64), ("C_sm", c_i64), ("C_sg", c_i64),
        ("initial_state", c_vp),
        ("y", c_vp), ("y_sb", c_i64), ("y_sl", c_i64), ("y_sm", c_i64), ("y_sh", c_i64),
        ("final_state", c_vp),
    ]


class Mamba1ScanArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("dim", c_i32), ("seqlen", c_i32), ("dstate", c_i32),
        ("u", c_vp), ("u_sb", c_i64), ("u_sd", c_i64), ("u_sl", c_i64),
        ("delta", c_vp), ("delta_sb", c_i64), ("delta_sd", c_i64), ("delta_sl", c_i64),
        ("A", c_vp), ("A_sd", c_i64), ("A_sn", c_i64),
        ("B", c_vp), ("B_sb", c_i64), ("B_sn", c_i64), ("B_sl", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sn", c_i64), ("C_sl", c_i64),
        ("D", c_vp),
        ("z", c_vp), ("z_sb", c_i64), ("z_sd", c_i64), ("z_sl", c_i64),
        ("delta_bias", c_vp), ("delta_softplus", c_i32),
        ("initial_state", c_vp),
        ("y", c_vp), ("y_sb", c_i64), ("y_sd", c_i64), ("y_sl", c_i64),
        ("final_state", c_vp),
    ]


class Mamba1StepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("dim", c_i32), ("dstate", c_i32),
        ("u", c_vp), ("u_sb", c_i64),
        ("delta", c_vp), ("delta_sb", c_i64),
        ("A", c_vp), ("A_sd", c_i64), ("A_sn", c_i64),
        ("B", c_vp), ("B_sb", c_i64), ("B_sn", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sn", c_i64),
        ("D", c_vp),
        ("z", c_vp), ("z_sb", c_i64),
        ("delta_bias", c_vp), ("delta_softplus", c_i32),
        ("state", c_vp),
        ("y", c_vp), ("y_sb", c_i64),
    ]


class Conv1dStepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("channels", c_i32), ("kernel", c_i32),
        ("x_dtype", c_i32), ("out_dtype", c_i32),
        ("x", c_vp), ("x_sb", c_i64),
        ("state", c_vp), ("w", c_vp), ("bias", c_vp),
        ("silu", c_i32),
        ("out", c_vp), ("out_sb", c_i64),
    ]


class Mamba3StepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("nheads", c_i32), ("headdim", c_i32), ("ngroups", c_i32),
        ("dstate", c_i32), ("mimo", c_i32), ("rope_dim", c_i32),
        ("proj_dtype", c_i32), ("out_dtype", c_i32),
        ("proj", c_vp), ("proj_sb", c_i64),
        ("ssm_state", c_vp), ("k_state", c_vp), ("v_state", c_vp), ("angle", c_vp),
        ("dt_bias", c_vp),
        ("a_floor", ctypes.c_float), ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float),
        ("rotation_range", ctypes.c_float),
        ("b_norm_w", c_vp), ("c_norm_w", c_vp), ("b_bias", c_vp), ("c_bias", c_vp),
        ("mimo_x", c_vp), ("mimo_z", c_vp), ("mimo_o", c_vp),
        ("D", c_vp), ("out_norm_w", c_vp),
        ("out", c_vp), ("out_sb", c_i64),
    ]


class Mamba3PrepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("nheads", c_i32), ("headdim", c_i32),
        ("ngroups", c_i32), ("dstate", c_i32), ("mimo", c_i32), ("rope_dim", c_i32),
        ("proj_dtype", c_i32), ("io_dtype", c_i32),
        ("proj", c_vp), ("proj_sb", c_i64), ("proj_sl", c_i64),
        ("ssm_state", c_vp), ("k_state", c_vp), ("v_state", c_vp), ("angle", c_vp), ("angle_out", c_vp),
        ("dt_bias", c_vp),
        ("a_floor", ctypes.c_float), ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float),
        ("rotation_range", ctypes.c_float),
        ("b_norm_w", c_vp), ("c_norm_w", c_vp), ("b_bias", c_vp), ("c_bias", c_vp), ("mimo_x", c_vp),
        ("v", c_vp), ("B", c_vp), ("C", c_vp),
        ("da", c_vp), ("gamma", c_vp), ("scale", c_vp), ("initial_state", c_vp),
    ]


class Ssd2BwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("nheads", c_i32), ("headdim", c_i32), ("ngroups", c_i32),
        ("dstate", c_i32),
        ("x", c_vp), ("x_sb", c_i64), ("x_sl", c_i64), ("x_sh", c_i64),
        ("dt", c_vp), ("dt_sb", c_i64), ("dt_sl", c_i64), ("dt_sh", c_i64),
        ("A", c_vp),
        ("B", c_vp), ("B_sb", c_i64), ("B_sl", c_i64), ("B_sg", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sl", c_i64), ("C_sg", c_i64),
        ("D", c_vp), ("initial_state", c_vp),
        ("dy", c_vp), ("dy_sb", c_i64), ("dy_sl", c_i64), ("dy_sh", c_i64),
        ("d_final_state", c_vp),
        ("dx", c_vp), ("ddt", c_vp), ("dA", c_vp), ("dB", c_vp), ("dC", c_vp), ("dD", c_vp),
        ("d_initial_state", c_vp),
    ]


class Ssd3BwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("mimo", c_i32), ("nheads", c_i32), ("headdim", c_i32),
        ("ngroups", c_i32), ("dstate", c_i32),
        ("v", c_vp), ("v_sb", c_i64), ("v_sl", c_i64), ("v_sm", c_i64), ("v_sh", c_i64),
        ("da", c_vp), ("da_sb", c_i64), ("da_sl", c_i64), ("da_sh", c_i64),
        ("gamma", c_vp), ("gamma_sb", c_i64), ("gamma_sl", c_i64), ("gamma_sh", c_i64),
        ("scale", c_vp), ("scale_sb", c_i64), ("scale_sl", c_i64), ("scale_sh", c_i64),
        ("B", c_vp), ("B_sb", c_i64), ("B_sl", c_i64), ("B_sm", c_i64), ("B_sg", c_i64),
        ("C", c_vp), ("C_sb", c_i64), ("C_sl", c_i64), ("C_sm", c_i64), ("C_sg", c_i64),
        ("initial_state", c_vp),
        ("dy", c_vp), ("dy_sb", c_i64), ("dy_sl", c_i64), ("dy_sm", c_i64), ("dy_sh", c_i64),
        ("d_final_state", c_vp),
        ("dv", c_vp), ("dda", c_vp), ("dgamma", c_vp), ("dscale", c_vp), ("dB", c_vp), ("dC", c_vp),
        ("d_initial_state", c_vp),
    ]


class Mamba3FusedArgs(ctypes.Structure):
    _fields_ = [("prep", Mamba3PrepArgs), ("D", c_vp), ("y", c_vp), ("final_state", c_vp)]


class Mamba3FinishArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("nheads", c_i32), ("headdim", c_i32), ("mimo", c_i32),
        ("io_dtype", c_i32), ("z_dtype", c_i32), ("out_dtype", c_i32),
        ("y_ssd", c_vp), ("v", c_vp),
        ("z", c_vp), ("z_sb", c_i64), ("z_sl", c_i64),
        ("D", c_vp), ("mimo_z", c_vp), ("mimo_o", c_vp), ("out_norm_w", c_vp),
        ("out", c_vp), ("out_sb", c_i64), ("out_sl", c_i64),
        ("y_ranks", c_i32),
    ]


class Mamba3DoubleInputsArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("nheads", c_i32), ("headdim", c_i32), ("ngroups", c_i32),
        ("dstate", c_i32), ("mimo", c_i32), ("proj_dtype", c_i32), ("io_dtype", c_i32),
        ("proj", c_vp), ("proj_sb", c_i64), ("proj_sl", c_i64),
        ("dt_bias", c_vp), ("a_floor", ctypes.c_float), ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float),
        ("v", c_vp), ("B", c_vp), ("C", c_vp),
        ("x_prev", c_vp), ("k_prev", c_vp), ("mimo_x", c_vp),
        ("v2", c_vp), ("B2", c_vp), ("C2", c_vp),
    ]


class Mamba2StepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("nheads", c_i32), ("headdim", c_i32), ("ngroups", c_i32),
        ("dstate", c_i32), ("conv_kernel", c_i32),
        ("zxbcdt_dtype", c_i32), ("out_dtype", c_i32), ("norm_before_gate", c_i32),
        ("zxbcdt", c_vp), ("zxbcdt_sb", c_i64),
        ("conv_state", c_vp), ("conv_w", c_vp), ("conv_b", c_vp),
        ("dt_bias", c_vp), ("A", c_vp), ("D", c_vp),
        ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float),
        ("norm_w", c_vp), ("ssm_state", c_vp),
        ("out", c_vp), ("out_sb", c_i64),
    ]


class RmsNormArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_i32), ("cols", c_i32), ("add_dtype", c_i32), ("out_dtype", c_i32),
        ("x", c_vp), ("x_sr", c_i64),
        ("add", c_vp), ("add_sr", c_i64),
        ("weight", c_vp),
        ("out", c_vp), ("out_sr", c_i64),
    ]


class Mamba2ConvArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("channels", c_i32), ("kernel", c_i32), ("nheads", c_i32),
        ("in_dtype", c_i32), ("out_dtype", c_i32),
        ("proj", c_vp), ("proj_sb", c_i64), ("proj_sl", c_i64),
        ("xbc_offset", c_i32), ("dt_offset", c_i32),
        ("conv_w", c_vp), ("conv_b", c_vp), ("conv_state", c_vp), ("dt_bias", c_vp),
        ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float),
        ("xbc", c_vp), ("xbc_sb", c_i64), ("xbc_sl", c_i64),
        ("dt", c_vp),
    ]


class Mamba2GatedNormArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("seqlen", c_i32), ("width", c_i32), ("norm_before_gate", c_i32),
        ("y_dtype", c_i32), ("z_dtype", c_i32), ("out_dtype", c_i32),
        ("eps", ctypes.c_float),
        ("y", c_vp), ("y_sb", c_i64), ("y_sl", c_i64),
        ("z", c_vp), ("z_sb", c_i64), ("z_sl", c_i64),
        ("gamma", c_vp),
        ("out", c_vp), ("out_sb", c_i64), ("out_sl", c_i64),
    ]


class LinearArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_i32), ("d_in", c_i32), ("d_out", c_i32), ("x_dtype", c_i32), ("y_dtype", c_i32),
        ("x", c_vp), ("x_ld", c_i64),
        ("packed_w", c_vp), ("bias", c_vp),
        ("y", c_vp), ("y_ld", c_i64),
    ]


class Mamba2LayerArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("d_model", c_i32), ("nheads", c_i32), ("headdim", c_i32), ("ngroups", c_i32),
        ("dstate", c_i32), ("conv_kernel", c_i32), ("norm_before_gate", c_i32), ("zxbcdt_dtype", c_i32),
        ("x", c_vp), ("x_sb", c_i64),
        ("pre_norm_w", c_vp), ("in_proj", c_vp), ("in_proj_b", c_vp), ("out_proj", c_vp), ("out_proj_b", c_vp),
        ("conv_state", c_vp), ("conv_w", c_vp), ("conv_b", c_vp),
        ("dt_bias", c_vp), ("A", c_vp), ("D", c_vp),
        ("dt_min", ctypes.c_float), ("dt_max", ctypes.c_float),
        ("norm_w", c_vp), ("ssm_state", c_vp), ("concurrent", c_i32),
    ]


# name -> (argtypes, restype); the exported symbol set of include/mamba_hip.h
_SIGNATURES = {
    "mamba_last_error": ([], ctypes.c_char_p),
    "mamba_version": ([], ctypes.c_char_p),
    "mamba_ssd2_workspace_size": ([ctypes.POINTER(Ssd2Args)], ctypes.c_size_t),
    "mamba_ssd2_fast_path": ([ctypes.POINTER(Ssd2Args)], ctypes.c_int),
    "mamba_ssd2_fwd": ([ctypes.POINTER(Ssd2Args), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd2_fwd_generic": ([ctypes.POINTER(Ssd2Args), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd2_fwd_timed": ([ctypes.POINTER(Ssd2Args), c_vp, ctypes.c_size_t, c_vp, c_vp, c_vp],
                             ctypes.c_int),
    "mamba_ssd2_bwd_workspace_size": ([ctypes.POINTER(Ssd2BwdArgs)], ctypes.c_size_t),
    "mamba_ssd2_bwd": ([ctypes.POINTER(Ssd2BwdArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd2_bwd_timed": ([ctypes.POINTER(Ssd2BwdArgs), c_vp, ctypes.c_size_t, c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba_ssd3_bwd_workspace_size": ([ctypes.POINTER(Ssd3BwdArgs)], ctypes.c_size_t),
    "mamba_ssd3_bwd": ([ctypes.POINTER(Ssd3BwdArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd3_bwd_timed": ([ctypes.POINTER(Ssd3BwdArgs), c_vp, ctypes.c_size_t, c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba_ssd3_workspace_size": ([ctypes.POINTER(Ssd3Args)], ctypes.c_size_t),
    "mamba_ssd3_fast_path": ([ctypes.POINTER(Ssd3Args)], ctypes.c_int),
    "mamba_ssd3_fwd": ([ctypes.POINTER(Ssd3Args), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd3_fwd_generic": ([ctypes.POINTER(Ssd3Args), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd3_fwd_timed": ([ctypes.POINTER(Ssd3Args), c_vp, ctypes.c_size_t, c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba_ssd3_double_workspace_size": ([ctypes.POINTER(Ssd3DoubleArgs)], ctypes.c_size_t),
    "mamba_ssd3_double_fast_path": ([ctypes.POINTER(Ssd3DoubleArgs)], ctypes.c_int),
    "mamba_ssd3_double_fwd": ([ctypes.POINTER(Ssd3DoubleArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba_ssd3_double_fwd_generic": ([ctypes.POINTER(Ssd3DoubleArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba1_scan_fwd": ([ctypes.POINTER(Mamba1ScanArgs), c_vp], ctypes.c_int),
    "mamba1_scan_fwd_timed": ([ctypes.POINTER(Mamba1ScanArgs), c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba1_scan_step": ([ctypes.POINTER(Mamba1StepArgs), c_vp], ctypes.c_int),
    "mamba3_step_ssm": ([ctypes.POINTER(Mamba3StepArgs), c_vp], ctypes.c_int),
    "mamba2_conv_fwd": ([ctypes.POINTER(Mamba2ConvArgs), c_vp], ctypes.c_int),
    "mamba2_gated_rmsnorm": ([ctypes.POINTER(Mamba2GatedNormArgs), c_vp], ctypes.c_int),
    "mamba3_prep_fast_path": ([ctypes.POINTER(Mamba3PrepArgs)], ctypes.c_int),
    "mamba3_prep_workspace_size": ([ctypes.POINTER(Mamba3PrepArgs)], ctypes.c_size_t),
    "mamba3_prep_fwd": ([ctypes.POINTER(Mamba3PrepArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba3_finish_fwd": ([ctypes.POINTER(Mamba3FinishArgs), c_vp], ctypes.c_int),
    "mamba3_ssd_fused_supported": ([ctypes.POINTER(Mamba3FusedArgs)], ctypes.c_int),
    "mamba3_ssd_fused_fwd": ([ctypes.POINTER(Mamba3FusedArgs), c_vp], ctypes.c_int),
    "mamba3_ssd_fused_fwd_timed": ([ctypes.POINTER(Mamba3FusedArgs), c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba3_double_inputs": ([ctypes.POINTER(Mamba3DoubleInputsArgs), c_vp], ctypes.c_int),
    "mamba3_step_ssm_timed": ([ctypes.POINTER(Mamba3StepArgs), c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba1_scan_step_timed": ([ctypes.POINTER(Mamba1StepArgs), c_vp, c_vp, c_vp], ctypes.c_int),
    "mamba_conv1d_step": ([ctypes.POINTER(Conv1dStepArgs), c_vp], ctypes.c_int),
    "mamba2_step_workspace_size": ([ctypes.POINTER(Mamba2StepArgs)], ctypes.c_size_t),
    "mamba2_step_ssm": ([ctypes.POINTER(Mamba2StepArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba2_step_ssm_timed": ([ctypes.POINTER(Mamba2StepArgs), c_vp, ctypes.c_size_t, c_vp, c_vp, c_vp],
                              ctypes.c_int),
    "mamba_rmsnorm": ([ctypes.POINTER(RmsNormArgs), c_vp], ctypes.c_int),
    "mamba_linear_packed_size": ([c_i32, c_i32], ctypes.c_size_t),
    "mamba_linear_pack": ([c_vp, c_i32, c_i32, c_i64, c_i32, c_vp, c_vp], ctypes.c_int),
    "mamba_linear_workspace_size": ([ctypes.POINTER(LinearArgs)], ctypes.c_size_t),
    "mamba_linear_fwd": ([ctypes.POINTER(LinearArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba2_layer_workspace_size": ([ctypes.POINTER(Mamba2LayerArgs)], ctypes.c_size_t),
    "mamba2_layer_step": ([ctypes.POINTER(Mamba2LayerArgs), c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba2_layer_step_timed": ([ctypes.POINTER(Mamba2LayerArgs), c_vp, ctypes.c_size_t, c_vp, c_vp, c_vp],
                                ctypes.c_int),
    "mamba2_stack_step": ([ctypes.POINTER(Mamba2LayerArgs), c_i32, c_vp, ctypes.c_size_t, c_vp], ctypes.c_int),
    "mamba2_stack_step_timed": ([ctypes.POINTER(Mamba2LayerArgs), c_i32, c_vp, ctypes.c_size_t, c_vp,
                                 ctypes.POINTER(c_vp), ctypes.POINTER(c_vp)], ctypes.c_int),
    "mamba2_stack_step_noalloc": ([ctypes.POINTER(Mamba2LayerArgs), c_i32, c_vp], ctypes.c_int),
}

_lib = None


def lib():
    """Load libmamba_hip.so once; raise if it is not built."""
    global _lib
    if _lib is None:
        path = os.path.normpath(LIB_PATH)
        if not os.path.exists(path):
            raise MambaHipError(
                f"{path} is not built; run `python burn-mamba_amd/build.py` (no CPU fallback exists)")
        L = ctypes.CDLL(path)
        for name, (argt, rest) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argt
            fn.restype = rest
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def check(status: int, what: str):
    if status != 0:
        msg = lib().mamba_last_error().decode(errors="replace")
        raise MambaHipError(f"{what} failed with status {status}: {msg}")
