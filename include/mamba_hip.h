/*
 * mamba_hip.h — C ABI of the MI355X (gfx950) SSM hot path for burn-mamba.
 *
 * One shared library, libmamba_hip.so, built from burn-mamba_amd/csrc/ with
 * hipcc --offload-arch=gfx950.  Every entry point:
 *   - takes plain device pointers, sizes and element strides (no framework types);
 *   - is stream-ordered on the hipStream_t it is given and returns without a
 *     host synchronisation;
 *   - validates shapes/pointers on the host first and returns a non-zero
 *     mamba_status (never launching a kernel) when they are wrong — the
 *     reference panics via assert! in the same places, the Rust binding maps a
 *     non-zero status back to a panic;
 *   - allocates nothing: scratch memory comes from a caller-owned workspace
 *     whose size the matching *_workspace_size() reports.
 * Calls that share a workspace buffer must be ordered on one stream.
 *
 * Reference interfaces replaced (swfsql/burn-mamba, paths relative to its root):
 *   mamba_ssd2_fwd      <- Mamba2BackendExt::ssd_serial_recalculated
 *                          (src/mamba2/ssd/serial_recalculated/serial_recalculated.rs:86-98),
 *                          reached from Mamba2SsdInput::run (src/mamba2/ssd/ssd_path.rs:149-155)
 *   mamba_ssd3_fwd      <- Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated
 *                          (src/mamba3/single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-114)
 *   mamba_ssd3_double_fwd <- Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated
 *                          (src/mamba3/double_ssd/ssd/serial_recalculated/serial_recalculated.rs:76-94)
 *   mamba1_scan_fwd     <- Mamba1::selective_scan (src/mamba1/mamba1.rs:422-430)
 *                          plus the silu(z) gate of Mamba1::forward (mamba1.rs:348)
 *   mamba1_scan_step    <- Mamba1::selective_scan_step (src/mamba1/mamba1.rs:666-733)
 *   mamba_conv1d_step   <- the conv-window step of Mamba1::step (src/mamba1/mamba1.rs:558-597)
 *   mamba3_step_ssm     <- Mamba3::step between in_proj and out_proj
 *                          (src/mamba3/double_ssd/double_ssd/mod.rs:634-760)
 *   mamba3_prep_fwd     <- Mamba3::forward_single_ssd steps 2-6, before the SSD seam
 *                          (src/mamba3/single_ssd/single_ssd/mod.rs:86-262)
 *   mamba3_finish_fwd   <- the same forward's step 9 before out_proj (:288-332)
 *   mamba3_double_inputs <- the gamma / beta inputs of Mamba3::forward_double_ssd
 *                          (src/mamba3/double_ssd/double_ssd/mod.rs:174-282), as one
 *                          2M-rank call of mamba_ssd3_double_fwd
 *   mamba2_step_ssm     <- the body of Mamba2::step between in_proj and out_proj
 *                          (src/mamba2/mamba2.rs:857-995)
 *   mamba_linear_fwd    <- burn::nn::Linear::forward in the decode steps (packed weights)
 *   mamba2_layer_step   <- Layer::step_one around Mamba2::step (src/modules/layer.rs:224-232,
 *                          src/mamba2/mamba2.rs:820-1004), with packed in_proj/out_proj
 *   mamba2_stack_step   <- Layers::step over such layers, without class latents
 *                          (src/modules/layers.rs:427)
 *   mamba_rmsnorm       <- RmsNorm::forward (src/modules/norm/rms_norm.rs:53-98), the
 *                          pre-norm and residual of Layer::step_one (src/modules/layer.rs:224-232)
 *   mamba2_conv_fwd     <- Mamba2::forward steps 2 and 4 (src/mamba2/mamba2.rs:618-699): causal
 *                          depthwise conv1d + SiLU over xBC, dt softplus/clamp, conv-cache update
 *   mamba2_gated_rmsnorm <- RmsNormGated::forward (src/modules/norm/rms_norm_gated.rs:70-135),
 *                          step 7 of Mamba2::forward (src/mamba2/mamba2.rs:776)
 */
#ifndef MAMBA_HIP_H
#define MAMBA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers (it is a pointer type). */
typedef struct ihipStream_t* mamba_stream_t;

typedef enum mamba_status {
    MAMBA_OK = 0,
    MAMBA_ERR_INVALID_ARG = 1,   /* bad shape, null required pointer, bad stride */
    MAMBA_ERR_UNSUPPORTED = 2,   /* valid request this build does not implement */
    MAMBA_ERR_WORKSPACE = 3,     /* workspace missing or smaller than *_workspace_size */
    MAMBA_ERR_HIP = 4            /* a HIP runtime call failed (see mamba_last_error) */
} mamba_status;

typedef enum mamba_dtype {
    MAMBA_F32 = 0,
    MAMBA_BF16 = 1
} mamba_dtype;

/* Human-readable description of the last error raised on the calling thread. */
const char* mamba_last_error(void);
/* Library version string ("mamba_hip <semver> gfx950"). */
const char* mamba_version(void);

/* ------------------------------------------------------------------------- */
/* Mamba-2 chunked SSD forward (K1 cumsum, K2 C.B^T, K3 chunk state, K4 state  */
/* passing, K5 chunk scan).                                                   */
/*                                                                             */
/*   y[b,t,h,:] = sum_{s<=t} (C_t . B_s) exp(sum_{s<k<=t} dt_k A_h) dt_s x_s    */
/*                + exp(sum_{k<=t} dt_k A_h) C_t . h0 + D_h x_t                 */
/*                                                                             */
/* Element strides are given for the three outer axes; the innermost axis      */
/* (headdim for x/y, dstate for B/C) must be contiguous.  Head h reads group   */
/* h / (nheads / ngroups) (src/modules/misc/gqa.rs:30-56); pass ngroups =      */
/* nheads for the reference's per-head-expanded B/C.  dt is the discretised    */
/* step (post softplus/clamp, src/mamba2/mamba2.rs:695) in f32; the reference  */
/* seam's dt_bhnl layout is expressed with dt strides.  seqlen need not be a   */
/* multiple of chunk_len: the tail behaves as the zero padding of              */
/* src/mamba2/mamba2.rs:709-722.                                               */
/* ------------------------------------------------------------------------- */
typedef struct mamba_ssd2_args {
    int32_t batch, seqlen, nheads, headdim, ngroups, dstate, chunk_len;
    int32_t io_dtype;                 /* mamba_dtype of x, B, C and y */
    const void* x;  int64_t x_sb, x_sl, x_sh;      /* [b, l, h, p]          */
    const float* dt; int64_t dt_sb, dt_sl, dt_sh;  /* [b, l, h] f32         */
    const float* A;                                 /* [h] f32, negative     */
    const void* B;  int64_t B_sb, B_sl, B_sg;      /* [b, l, g, n]          */
    const void* C;  int64_t C_sb, C_sl, C_sg;      /* [b, l, g, n]          */
    const float* D;                                 /* [h] f32 or NULL (=0)  */
    const float* initial_state;                     /* [b, h, p, n] f32 or NULL */
    const float* init_state_hpr;                    /* [h, p, n] f32 or NULL (learnable h0) */
    void* y;        int64_t y_sb, y_sl, y_sh;      /* [b, l, h, p]          */
    float* final_state;                             /* [b, h, p, n] f32      */
} mamba_ssd2_args;

size_t mamba_ssd2_workspace_size(const mamba_ssd2_args* args);
/* 1 if mamba_ssd2_fwd takes the MFMA fast path for these arguments (bf16     */
/* I/O, headdim 64, dstate 64 or 128, chunk_len a multiple of 32 up to 256,   */
/* 16-byte aligned rows), 0 if it takes the shape-generic path, -1 if the     */
/* arguments are invalid.  No counterpart in the reference (its backends have  */
/* a single code path per op).                                                */
int mamba_ssd2_fast_path(const mamba_ssd2_args* args);
int mamba_ssd2_fwd(const mamba_ssd2_args* args, void* workspace, size_t workspace_bytes,
                   mamba_stream_t stream);

/* Same contract, forced onto the shape-generic kernels (no MFMA fast path);    */
/* used to cross-check the fast path.                                           */
int mamba_ssd2_fwd_generic(const mamba_ssd2_args* args, void* workspace, size_t workspace_bytes,
                           mamba_stream_t stream);

/* Same as mamba_ssd2_fwd, and additionally records the caller's HIP events   */
/* (hipEvent_t, already created) on `stream` immediately before and after the  */
/* dominant kernel of the call (the chunk-scan kernel), so a benchmark can     */
/* time that kernel alone with hipEventElapsedTime.  No counterpart in the    */
/* reference (its benches time whole blocks, benches/layer.rs:176-187).        */
int mamba_ssd2_fwd_timed(const mamba_ssd2_args* args, void* workspace, size_t workspace_bytes,
                         mamba_stream_t stream, void* event_start, void* event_stop);

/* ------------------------------------------------------------------------- */
/* Mamba-2 SSD backward (recompute form): the gradients of mamba_ssd2_fwd's    */
/* y and final state with respect to x, dt, A, B, C, D and the initial state,  */
/* given dy and d(final state).  Replaces the Autodiff arm of                  */
/* Mamba2BackendExt::ssd_serial_recalculated                                   */
/* (src/mamba2/ssd/serial_recalculated/backward.rs:29-321) and its gradient   */
/* math, combined_backward (combined_backward.rs:126-593): the forward's chunk */
/* states are recomputed into the workspace, then a reverse chunk loop         */
/* carries the state gradient.  f32 inputs and gradients; layouts and strides  */
/* as mamba_ssd2_args; dB / dC are per group (summed over the group's heads in */
/* head order; with ngroups = nheads they are per head, as the reference's    */
/* expanded B / C).  init_state_hpr is not supported (the reference's serial  */
/* path asserts it absent, src/mamba2/ssd/serial.rs:48-51).  headdim x dstate */
/* <= 8192.  Deterministic (no atomics).                                       */
/* ------------------------------------------------------------------------- */
typedef struct mamba_ssd2_bwd_args {
    int32_t batch, seqlen, nheads, headdim, ngroups, dstate;
    const float* x;  int64_t x_sb, x_sl, x_sh;      /* [b, l, h, p]           */
    const float* dt; int64_t dt_sb, dt_sl, dt_sh;   /* [b, l, h]              */
    const float* A;                                  /* [h]                    */
    const float* B;  int64_t B_sb, B_sl, B_sg;      /* [b, l, g, n]           */
    const float* C;  int64_t C_sb, C_sl, C_sg;      /* [b, l, g, n]           */
    const float* D;                                  /* [h] or NULL (= 0)      */
    const float* initial_state;                      /* [b, h, p, n] or NULL   */
    const float* dy; int64_t dy_sb, dy_sl, dy_sh;   /* [b, l, h, p]           */
    const float* d_final_state;                      /* [b, h, p, n] or NULL   */
    float* dx;                                       /* [b, l, h, p] contiguous */
    float* ddt;                                      /* [b, l, h] contiguous   */
    float* dA;                                       /* [h]                    */
    float* dB;                                       /* [b, l, g, n] contiguous */
    float* dC;                                       /* [b, l, g, n] contiguous */
    float* dD;                                       /* [h] or NULL            */
    float* d_initial_state;                          /* [b, h, p, n]           */
} mamba_ssd2_bwd_args;

/* Workspace bytes (chunk states, per-head dB / dC when ngroups < nheads,     */
/* per-(batch, head) partial sums); 0 if the arguments are invalid.            */
size_t mamba_ssd2_bwd_workspace_size(const mamba_ssd2_bwd_args* args);
int mamba_ssd2_bwd(const mamba_ssd2_bwd_args* args, void* workspace, size_t workspace_bytes,
                   mamba_stream_t stream);
/* Same, recording the caller's HIP events immediately before and after the   */
/* dominant kernel (the reverse chunk loop).  No counterpart in the reference. */
int mamba_ssd2_bwd_timed(const mamba_ssd2_bwd_args* args, void* workspace, size_t workspace_bytes,
                         mamba_stream_t stream, void* event_start, void* event_stop);

/* ------------------------------------------------------------------------- */
/* Mamba-3 single-pass chunked SSD forward (trapezoidal discretisation, MIMO   */
/* rank M fused into the time axis):                                           */
/*                                                                             */
/*   y[t,mo] = exp(cs_t) C[t,mo].h_in                                          */
/*           + sum_{t'<t, mi} (C[t,mo].B[t',mi]) exp(cs_t - cs_t') scale_t' v[t',mi] */
/*           + gamma_t sum_mi (C[t,mo].B[t,mi]) v[t,mi]                        */
/*   h_out   = exp(cs_end) h_in + sum_{t,mi} exp(cs_end - cs_t) scale_t v[t,mi] (x) B[t,mi] */
/*                                                                             */
/* with cs the within-chunk cumulative sum of da = dt A.  Replaces            */
/* Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated                   */
/* (src/mamba3/single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-114),*/
/* whose [b, n, l, ...] chunked tensors are the [b, l, ...] tensors here       */
/* (chunk_len = l); B/C are per head there (ngroups = nheads).  Strides are    */
/* element strides; the innermost axis (headdim, dstate) is contiguous.  The   */
/* reference has no D term in this seam.                                       */
/* ------------------------------------------------------------------------- */
typedef struct mamba_ssd3_args {
    int32_t batch, seqlen, mimo, nheads, headdim, ngroups, dstate, chunk_len;
    int32_t io_dtype;                                      /* v, B, C, y           */
    const void* v;      int64_t v_sb, v_sl, v_sm, v_sh;      /* [b, l, m, h, p]      */
    const float* da;    int64_t da_sb, da_sl, da_sh;         /* [b, l, h]  dt * A    */
    const float* gamma; int64_t gamma_sb, gamma_sl, gamma_sh; /* [b, l, h]           */
    const float* scale; int64_t scale_sb, scale_sl, scale_sh; /* [b, l, h]           */
    const void* B;      int64_t B_sb, B_sl, B_sm, B_sg;      /* [b, l, m, g, n]      */
    const void* C;      int64_t C_sb, C_sl, C_sm, C_sg;      /* [b, l, m, g, n]      */
    const float* initial_state;                              /* [b, h, p, n] or NULL */
    void* y;            int64_t y_sb, y_sl, y_sm, y_sh;      /* [b, l, m, h, p]      */
    float* final_state;                                      /* [b, h, p, n] f32     */
} mamba_ssd3_args;

size_t mamba_ssd3_workspace_size(const mamba_ssd3_args* args);
/* 1 if mamba_ssd3_fwd takes the single-kernel MFMA fast path (bf16 I/O,       */
/* headdim 64, dstate 128, mimo dividing 32, fused (l, m) axis of uniform      */
/* stride, 16-byte aligned rows), 0 for the shape-generic path, -1 if the      */
/* arguments are invalid.  The fast path chunks on 128 fused positions         */
/* whatever chunk_len says (the chunked form is exact for any chunk length)    */
/* and needs no workspace.  No counterpart in the reference.                   */
int mamba_ssd3_fast_path(const mamba_ssd3_args* args);
int mamba_ssd3_fwd(const mamba_ssd3_args* args, void* workspace, size_t workspace_bytes, mamba_stream_t stream);
/* Same contract, forced onto the shape-generic kernels; used to cross-check   */
/* the fast path.                                                              */
int mamba_ssd3_fwd_generic(const mamba_ssd3_args* args, void* workspace, size_t workspace_bytes,
                           mamba_stream_t stream);
/* As mamba_ssd3_fwd, recording the caller's HIP events around the chunk-scan  */
/* kernel (benchmark timing; no counterpart in the reference).                 */
int mamba_ssd3_fwd_timed(const mamba_ssd3_args* args, void* workspace, size_t workspace_bytes,
                         mamba_stream_t stream, void* event_start, void* event_stop);

/* ---- Mamba-3 double SSD (the Mamba3DoubleSsdBackendExt seam) ------------- */
/* Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated                   */
/* (src/mamba3/double_ssd/ssd/serial_recalculated/serial_recalculated.rs:76-94; */
/* K1-K5 in src/mamba3/double_ssd/ssd/serial.rs:118-409): v, da, B, C, h0 ->  */
/* y, final state, with the same chunk axis folding and strides as            */
/* mamba_ssd3_args.  v arrives pre-scaled (no scale or gamma column), and the */
/* fused-rank causal mask keeps every rank pair of the same step (triu(1) on  */
/* steps): y[t, m] = C[t, m] . h_t with h_t = exp(da_t) h_{t-1} +             */
/* sum_m' v[t, m'] (x) B[t, m'].  The single-SSD kernels run it with unit     */
/* coefficients; the fast-path conditions are those of mamba_ssd3_fwd.        */
typedef struct mamba_ssd3_double_args {
    int32_t batch, seqlen, mimo, nheads, headdim, ngroups, dstate, chunk_len;
    int32_t io_dtype;                                      /* v, B, C, y           */
    const void* v;      int64_t v_sb, v_sl, v_sm, v_sh;      /* [b, l, m, h, p]      */
    const float* da;    int64_t da_sb, da_sl, da_sh;         /* [b, l, h]  dt * A    */
    const void* B;      int64_t B_sb, B_sl, B_sm, B_sg;      /* [b, l, m, g, n]      */
    const void* C;      int64_t C_sb, C_sl, C_sm, C_sg;      /* [b, l, m, g, n]      */
    const float* initial_state;                              /* [b, h, p, n] or NULL */
    void* y;            int64_t y_sb, y_sl, y_sm, y_sh;      /* [b, l, m, h, p]      */
    float* final_state;                                      /* [b, h, p, n] f32     */
} mamba_ssd3_double_args;

size_t mamba_ssd3_double_workspace_size(const mamba_ssd3_double_args* args);
/* 1 / 0 / -1 as mamba_ssd3_fast_path.  No counterpart in the reference.       */
int mamba_ssd3_double_fast_path(const mamba_ssd3_double_args* args);
int mamba_ssd3_double_fwd(const mamba_ssd3_double_args* args, void* workspace, size_t workspace_bytes,
                          mamba_stream_t stream);
/* Same contract, forced onto the shape-generic kernels (cross-checks).        */
int mamba_ssd3_double_fwd_generic(const mamba_ssd3_double_args* args, void* workspace,
                                  size_t workspace_bytes, mamba_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Mamba-3 SSD backward (recompute form): the gradients of mamba_ssd3_fwd's    */
/* y and final state with respect to v, da, B, C, gamma, scale and the        */
/* initial state, given dy and d(final state).  Replaces the Autodiff arm of  */
/* Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated                   */
/* (src/mamba3/single_ssd/ssd/serial_recalculated/backward.rs:27-299; its      */
/* gradient math combined_backward.rs:74-536).  With gamma = scale = NULL     */
/* (unit weights; dgamma / dscale NULL) it is the Autodiff arm of             */
/* Mamba3DoubleSsdBackendExt::double_ssd_serial_recalculated                   */
/* (double_ssd/ssd/serial_recalculated/backward.rs:27-275, combined_backward.rs:98-542), */
/* whose forward (mamba_ssd3_double_fwd) is the single one with unit weights.  */
/* f32; element strides with the innermost axis contiguous; B / C in group    */
/* form (dB / dC summed over each group's heads).  mimo must divide 32.       */
/* headdim x dstate <= 8192.  Deterministic (no atomics).                      */
/* ------------------------------------------------------------------------- */
typedef struct mamba_ssd3_bwd_args {
    int32_t batch, seqlen, mimo, nheads, headdim, ngroups, dstate;
    const float* v;     int64_t v_sb, v_sl, v_sm, v_sh;           /* [b, l, m, h, p]      */
    const float* da;    int64_t da_sb, da_sl, da_sh;              /* [b, l, h]            */
    const float* gamma; int64_t gamma_sb, gamma_sl, gamma_sh;     /* [b, l, h] or NULL    */
    const float* scale; int64_t scale_sb, scale_sl, scale_sh;     /* [b, l, h] or NULL    */
    const float* B;     int64_t B_sb, B_sl, B_sm, B_sg;           /* [b, l, m, g, n]      */
    const float* C;     int64_t C_sb, C_sl, C_sm, C_sg;           /* [b, l, m, g, n]      */
    const float* initial_state;                                   /* [b, h, p, n] or NULL */
    const float* dy;    int64_t dy_sb, dy_sl, dy_sm, dy_sh;       /* [b, l, m, h, p]      */
    const float* d_final_state;                                   /* [b, h, p, n] or NULL */
    float* dv;                                                    /* [b, l, m, h, p] contiguous */
    float* dda;                                                   /* [b, l, h] contiguous */
    float* dgamma;                                                /* [b, l, h] or NULL    */
    float* dscale;                                                /* [b, l, h] or NULL    */
    float* dB;                                                    /* [b, l, m, g, n] contiguous */
    float* dC;                                                    /* [b, l, m, g, n] contiguous */
    float* d_initial_state;                                       /* [b, h, p, n]         */
} mamba_ssd3_bwd_args;

/* Workspace bytes (chunk states; per-head dB / dC when ngroups < nheads);     */
/* 0 if the arguments are invalid.                                             */
size_t mamba_ssd3_bwd_workspace_size(const mamba_ssd3_bwd_args* args);
int mamba_ssd3_bwd(const mamba_ssd3_bwd_args* args, void* workspace, size_t workspace_bytes,
                   mamba_stream_t stream);
/* Same, recording the caller's HIP events immediately before and after the   */
/* dominant kernel (the reverse chunk loop).  No counterpart in the reference. */
int mamba_ssd3_bwd_timed(const mamba_ssd3_bwd_args* args, void* workspace, size_t workspace_bytes,
                         mamba_stream_t stream, void* event_start, void* event_stop);

/* ------------------------------------------------------------------------- */
/* Mamba-1 selective scan (f32), with the optional dt bias + softplus of       */
/* Mamba1::ssm and the silu(z) gate of Mamba1::forward:                        */
/*                                                                             */
/*   dl = softplus(delta + delta_bias)  (or delta as given)                   */
/*   h[b,d,n] <- exp(dl A[d,n]) h[b,d,n] + dl B[b,n,t] u[b,d,t]                */
/*   y[b,d,t]  = (sum_n C[b,n,t] h[b,d,n] + D[d] u[b,d,t]) * silu(z[b,d,t])    */
/*                                                                             */
/* Every tensor is addressed through element strides, so both the reference's */
/* layouts (u,y [b,l,d]; delta [l,b,d]; B [b,l,n]; C [l,b,n]) and the         */
/* channel-major [b,d,l] / [b,n,l] layouts are accepted.  softplus(x) is      */
/* evaluated as x above 20 (where it equals x in f32); the reference's Burn   */
/* softplus returns inf above ~88.7.  Replaces Mamba1::selective_scan         */
/* (src/mamba1/mamba1.rs:422-523) and, with delta_bias/delta_softplus/z, the  */
/* scan part of Mamba1::ssm + the gate of Mamba1::forward (mamba1.rs:348,      */
/* 391-394).                                                                   */
/* ------------------------------------------------------------------------- */
typedef struct mamba1_scan_args {
    int32_t batch, dim, seqlen, dstate;
    const float* u;     int64_t u_sb, u_sd, u_sl;          /* [b, d, l]            */
    const float* delta; int64_t delta_sb, delta_sd, delta_sl;
    const float* A;     int64_t A_sd, A_sn;                /* [d, n]               */
    const float* B;     int64_t B_sb, B_sn, B_sl;          /* [b, n, l]            */
    const float* C;     int64_t C_sb, C_sn, C_sl;          /* [b, n, l]            */
    const float* D;                                         /* [d] or NULL          */
    const float* z;     int64_t z_sb, z_sd, z_sl;          /* [b, d, l] or NULL    */
    const float* delta_bias;                                /* [d] or NULL          */
    int32_t delta_softplus;                                 /* 0 or 1               */
    const float* initial_state;                             /* [b, d, n] or NULL    */
    float* y;           int64_t y_sb, y_sd, y_sl;          /* [b, d, l]            */
    float* final_state;                                     /* [b, d, n] or NULL    */
} mamba1_scan_args;

int mamba1_scan_fwd(const mamba1_scan_args* args, mamba_stream_t stream);
/* As mamba1_scan_fwd, recording the caller's HIP events around the scan      */
/* kernel (benchmark timing; no counterpart in the reference).                */
int mamba1_scan_fwd_timed(const mamba1_scan_args* args, mamba_stream_t stream, void* event_start,
                          void* event_stop);

/* ------------------------------------------------------------------------- */
/* Mamba-1 recurrent decode step (f32), one token per sequence:                */
/*                                                                             */
/*   dl = softplus(delta + delta_bias)  (or delta as given)                   */
/*   state[b,d,n] <- exp(dl A[d,n]) state[b,d,n] + (dl B[b,n]) u[b,d]          */
/*   y[b,d] = (sum_n state[b,d,n] C[b,n] + D[d] u[b,d]) * silu(z[b,d])          */
/*                                                                             */
/* Replaces Mamba1::selective_scan_step (src/mamba1/mamba1.rs:666-733); with   */
/* delta_bias/delta_softplus/z it also covers the dt_proj bias + softplus of   */
/* Mamba1::ssm_step (mamba1.rs:646) and the silu(res) gate of Mamba1::step     */
/* (mamba1.rs:603).  state is Mamba1Cache::ssm_bir (src/mamba1/cache.rs:30-47),*/
/* contiguous, updated in place.  softplus is evaluated as in mamba1_scan_fwd. */
/* ------------------------------------------------------------------------- */
typedef struct mamba1_step_args {
    int32_t batch, dim, dstate;
    const float* u;     int64_t u_sb;                /* [b, d]               */
    const float* delta; int64_t delta_sb;            /* [b, d]               */
    const float* A;     int64_t A_sd, A_sn;          /* [d, n]               */
    const float* B;     int64_t B_sb, B_sn;          /* [b, n]               */
    const float* C;     int64_t C_sb, C_sn;          /* [b, n]               */
    const float* D;                                  /* [d] or NULL          */
    const float* z;     int64_t z_sb;                /* [b, d] or NULL       */
    const float* delta_bias;                         /* [d] or NULL          */
    int32_t delta_softplus;                          /* 0 or 1               */
    float* state;                                    /* [b, d, n], in/out    */
    float* y;           int64_t y_sb;                /* [b, d]               */
} mamba1_step_args;

int mamba1_scan_step(const mamba1_step_args* args, mamba_stream_t stream);
/* As mamba1_scan_step, recording the caller's HIP events (already created)    */
/* on `stream` immediately around the kernel, for benchmark timing.  No       */
/* counterpart in the reference.                                              */
int mamba1_scan_step_timed(const mamba1_step_args* args, mamba_stream_t stream, void* event_start,
                           void* event_stop);

/* ------------------------------------------------------------------------- */
/* Depthwise causal conv, one step (the conv-window roll of Mamba1::step,      */
/* src/mamba1/mamba1.rs:558-597; Mamba-2's is fused into mamba2_step_ssm):     */
/*   state[b,c,:] <- (state[b,c,1:], x[b,c])                                   */
/*   out[b,c] = act(sum_k state[b,c,k] w[c,k] + bias[c]),  act = SiLU or id    */
/* state is Mamba1Cache::conv_bik [b, c, K] f32, contiguous, in place.          */
/* ------------------------------------------------------------------------- */
typedef struct mamba_conv1d_step_args {
    int32_t batch, channels, kernel;
    int32_t x_dtype, out_dtype;        /* mamba_dtype                            */
    const void* x;  int64_t x_sb;      /* [b, c] new column                      */
    float* state;                      /* [b, c, K], in/out                      */
    const float* w;                    /* [c, K] (Conv1d weight [c, 1, K])       */
    const float* bias;                 /* [c] or NULL                            */
    int32_t silu;                      /* 1: SiLU after the bias                 */
    void* out;      int64_t out_sb;    /* [b, c]                                 */
} mamba_conv1d_step_args;

int mamba_conv1d_step(const mamba_conv1d_step_args* args, mamba_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Mamba-3 decode step: everything of Mamba3::step between in_proj and         */
/* out_proj, per token (Complex2D rotation).  Replaces Mamba3::step_double_ssd */
/* (src/mamba3/double_ssd/double_ssd/mod.rs:634-760; single-SSD decoding uses  */
/* the same step, single_ssd/single_ssd/mod.rs:383-397) from the split of the  */
/* in_proj row to the MIMO merge: trapezoid coefficients (helpers.rs:42-73),   */
/* QK-norm + GQA + bias (helpers.rs:82-95), the cumulative-angle RoPE of B/C   */
/* (rotation/mod.rs:729-763, rope.rs:23-170), the state update                 */
/*   h = alpha h + sum_m gamma (x mimo_x[m]) (x) B[m] + sum_m beta (x_prev mimo_x[m]) (x) K[m] */
/* the readout sum_n C h + D v, and step_finish's gate / gated RMSNorm and     */
/* mimo_o merge (mod.rs:556-628).  The in_proj row is                          */
/*   [z (H P) | x (H P) | b_raw (M, G, N) | c_raw (M, G, N) | dd_dt (H) |      */
/*    dd_a (H) | lambda (H) | rot (A)],  A = max(rope_dim / 2, 1).             */
/* The four cache tensors (Mamba3DoubleSsdCache / Mamba3SingleSsdCache,        */
/* double_ssd/cache.rs:81-106) are updated in place: ssm, k_state = the        */
/* rotated B, v_state = x, angle = the wrapped cumulative angle.               */
/* dstate in {8, 16, 32, 64, 128, 256}, headdim * dstate <= 8192,              */
/* mimo in {1, 2, 4, 8}.                                                       */
/* ------------------------------------------------------------------------- */
typedef struct mamba3_step_args {
    int32_t batch, nheads, headdim, ngroups, dstate, mimo, rope_dim;
    int32_t proj_dtype, out_dtype;
    const void* proj;   int64_t proj_sb;             /* [b, row] in_proj output   */
    float* ssm_state;                                /* [b, H, P, N] in/out       */
    float* k_state;                                  /* [b, M, H, N] in/out       */
    float* v_state;                                  /* [b, H, P]    in/out       */
    float* angle;                                    /* [b, H, A]    in/out       */
    const float* dt_bias;                            /* [H]                       */
    float a_floor, dt_min, dt_max, rotation_range;
    const float* b_norm_w; const float* c_norm_w;    /* [N] QK-norm gammas        */
    const float* b_bias;   const float* c_bias;      /* [H, M, N]                 */
    const float* mimo_x; const float* mimo_z; const float* mimo_o; /* [H, M, P]; NULL if mimo == 1 */
    const float* D;                                  /* [H] or NULL               */
    const float* out_norm_w;                         /* [P] or NULL: gated RMSNorm instead of the silu gate */
    void* out;          int64_t out_sb;              /* [b, H P] (before out_proj) */
} mamba3_step_args;

int mamba3_step_ssm(const mamba3_step_args* args, mamba_stream_t stream);
/* As mamba3_step_ssm, recording the caller's HIP events around the kernel     */
/* (benchmark timing; no counterpart in the reference).                        */
int mamba3_step_ssm_timed(const mamba3_step_args* args, mamba_stream_t stream, void* event_start,
                          void* event_stop);

/* ------------------------------------------------------------------------- */
/* Mamba-3 prefill prologue: forward_single_ssd steps 2-6                      */
/* (src/mamba3/single_ssd/single_ssd/mod.rs:86-262) from the in_proj output to */
/* the inputs of mamba_ssd3_fwd: trapezoid coefficients (helpers.rs:42-73),    */
/* scale_t = gamma_t + (1 - lambda_{t+1}) dt_{t+1} (:129-150), QK-norm + GQA + */
/* bias (helpers.rs:82-95), the cumulative-angle RoPE of B and C               */
/* (rotate_bc_forward Complex2D, rotation/mod.rs:653-679), v = x mimo_x, and   */
/* the beta-seeded initial state ssm + (dt_0 - gamma_0) sum_m v_prev[m] (x)    */
/* K_prev[m] (:195-225).  The cache's k_state / v_state are replaced by this   */
/* call's last token (rotated B, x); the wrapped last angle goes to angle_out  */
/* (not aliasing angle).  The cache's ssm_state is read only: mamba_ssd3_fwd's */
/* final state is the new one.  proj row layout as for mamba3_step_ssm.        */
/* ------------------------------------------------------------------------- */
typedef struct mamba3_prep_args {
    int32_t batch, seqlen, nheads, headdim, ngroups, dstate, mimo, rope_dim;
    int32_t proj_dtype, io_dtype;                    /* io: v, B, C                */
    const void* proj;   int64_t proj_sb, proj_sl;    /* [b, l, row]                */
    const float* ssm_state;                          /* [b, H, P, N] (read)        */
    float* k_state;                                  /* [b, M, H, N] in/out        */
    float* v_state;                                  /* [b, H, P]    in/out        */
    const float* angle;                              /* [b, H, A]    in            */
    float* angle_out;                                /* [b, H, A]    out           */
    const float* dt_bias;                            /* [H]                        */
    float a_floor, dt_min, dt_max, rotation_range;
    const float* b_norm_w; const float* c_norm_w;    /* [N]                        */
    const float* b_bias;   const float* c_bias;      /* [H, M, N]                  */
    const float* mimo_x;                             /* [H, M, P]; NULL if mimo == 1 */
    void* v;                                         /* [b, l, M, H, P] out        */
    void* B;            void* C;                     /* [b, l, M, H, N] out        */
    float* da;          float* gamma;  float* scale; /* [b, l, H] out              */
    float* initial_state;                            /* [b, H, P, N] out           */
} mamba3_prep_args;

/* 1 if mamba3_prep_fwd runs the segment-parallel kernels (proj rows of 8k    */
/* elements at a 16-byte aligned base, headdim a multiple of 4, aligned        */
/* parameter and output buffers), 0 for the per-(batch, head, rank) kernel,    */
/* -1 if the arguments are invalid.                                            */
int mamba3_prep_fast_path(const mamba3_prep_args* args);
/* Workspace bytes mamba3_prep_fwd needs: per-segment angle totals (f64) when */
/* the sequence spans more than one 256-position segment, else 0.             */
size_t mamba3_prep_workspace_size(const mamba3_prep_args* args);
int mamba3_prep_fwd(const mamba3_prep_args* args, void* workspace, size_t workspace_bytes,
                    mamba_stream_t stream);

/* Mamba-3 prefill epilogue: forward_single_ssd step 9 before out_proj         */
/* (single_ssd/single_ssd/mod.rs:288-332): y += D v, the silu gate (or the     */
/* per-head gated RMSNorm) with z mimo_z[m], and the mimo_o merge over ranks.  */
typedef struct mamba3_finish_args {
    int32_t batch, seqlen, nheads, headdim, mimo;
    int32_t io_dtype, z_dtype, out_dtype;
    const void* y_ssd;                               /* [b, l, M, H, P] contiguous */
    const void* v;                                   /* [b, l, M, H, P] contiguous; */
                                                     /* may be NULL when D is NULL  */
    const void* z;      int64_t z_sb, z_sl;          /* [b, l, H P]                */
    const float* D;                                  /* [H] or NULL                */
    const float* mimo_z; const float* mimo_o;        /* [H, M, P]; NULL if mimo == 1 */
    const float* out_norm_w;                         /* [P] or NULL                */
    void* out;          int64_t out_sb, out_sl;      /* [b, l, H P]                */
    int32_t y_ranks;    /* ranks in y_ssd's rank axis, of which the first mimo are */
                        /* read (0 = mimo; 2 mimo for the double pathway's call)   */
} mamba3_finish_args;

int mamba3_finish_fwd(const mamba3_finish_args* args, mamba_stream_t stream);

/* Mamba-3 prefill prologue fused into the single SSD: forward_single_ssd      */
/* steps 2-7 and the D skip of step 9 (single_ssd/single_ssd/mod.rs:86-290) in */
/* one scan kernel (after the beta-seed kernel of mamba3_prep_fwd).  The scan  */
/* reads the raw in_proj row (x, group-form B / C, dd_dt, dd_A, lambda, the    */
/* rotation channels) and forms, in its B / C tile loaders, the trapezoid      */
/* coefficients, the QK-norm + bias, the cumulative-angle rotation and         */
/* v = x mimo_x; no per-head v / B / C / coefficient tensor reaches HBM.       */
/* Its output is y_ssd + D v per rank, for mamba3_finish_fwd with D = NULL.    */
/* prep: the prologue's arguments as for mamba3_prep_fwd, except that its v,   */
/* B, C, da, gamma and scale outputs are not used (may be NULL); its          */
/* initial_state receives the seeded state; the cache tail (k_state, v_state, */
/* angle_out) is written as by mamba3_prep_fwd.  Only the fast shape is       */
/* provided (bf16 proj and y, headdim 64, dstate 128, mimo 2 / 4 / 8, 16-byte */
/* aligned proj rows): mamba3_ssd_fused_supported says whether it applies;    */
/* otherwise run mamba3_prep_fwd -> mamba_ssd3_fwd -> mamba3_finish_fwd.  No   */
/* single counterpart in the reference (it replaces that sequence).           */
typedef struct mamba3_fused_args {
    mamba3_prep_args prep;
    const float* D;                                  /* [H] or NULL                */
    void* y;                                         /* [b, l, M, H, P] bf16 out,  */
                                                     /* contiguous                 */
    float* final_state;                              /* [b, H, P, N] f32 out; may  */
                                                     /* alias prep.ssm_state       */
} mamba3_fused_args;

/* 1 if mamba3_ssd_fused_fwd runs for these arguments, 0 if the shape or      */
/* layout is not the fused kernel's, -1 if the arguments are invalid.         */
int mamba3_ssd_fused_supported(const mamba3_fused_args* args);
int mamba3_ssd_fused_fwd(const mamba3_fused_args* args, mamba_stream_t stream);
/* As mamba3_ssd_fused_fwd, recording the caller's HIP events around the      */
/* seed and scan kernels (benchmark timing).                                   */
int mamba3_ssd_fused_fwd_timed(const mamba3_fused_args* args, mamba_stream_t stream, void* event_start,
                               void* event_stop);

/* Mamba-3 double-SSD pathway (Mamba3::forward_double_ssd,                     */
/* src/mamba3/double_ssd/double_ssd/mod.rs:40-369): its gamma call (gamma_t v_t, */
/* B_t, the cached state) and its beta call (beta_t v_{t-1}, B_{t-1}, with the  */
/* cache's x_prev mimo_x and K_prev at t = 0, zero state) share da and C, so   */
/* their sum is one mamba_ssd3_double_fwd over 2M ranks:                       */
/*   v2 = [gamma v | beta v_prev], B2 = [B | B_prev], C2 = [C | C]             */
/* whose first M ranks of y are y_gamma + y_beta and whose final state is the  */
/* sum of both.  This entry builds v2, B2, C2 from the prep's v, B, C (the    */
/* single-pathway prep computes the same normed, biased, rotated B/C) and the */
/* cache tail as it was before the prep; gamma and beta come from the in_proj */
/* row (trapezoidal_coefficients, helpers.rs:42-73).                           */
typedef struct mamba3_double_inputs_args {
    int32_t batch, seqlen, nheads, headdim, ngroups, dstate, mimo;
    int32_t proj_dtype, io_dtype;                    /* proj; v/B/C and outputs  */
    const void* proj;   int64_t proj_sb, proj_sl;    /* [b, l, d_in_proj]        */
    const float* dt_bias;                            /* [H]                      */
    float a_floor, dt_min, dt_max;
    const void* v; const void* B; const void* C;     /* [b, l, M, H, P|N] contig. */
    const float* x_prev;                             /* [b, H, P] before the prep */
    const float* k_prev;                             /* [b, M, H, N] before the prep */
    const float* mimo_x;                             /* [H, M, P] or NULL (M = 1) */
    void* v2; void* B2; void* C2;                    /* [b, l, 2M, H, P|N] contig. */
} mamba3_double_inputs_args;

int mamba3_double_inputs(const mamba3_double_inputs_args* args, mamba_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Mamba-2 recurrent decode step: everything of Mamba2::step between in_proj  */
/* and out_proj (src/mamba2/mamba2.rs:857-995), for one token per sequence:    */
/*                                                                             */
/*   zxbcdt = [z (d_inner) | xBC (conv_dim) | dt_raw (nheads)]  (in_proj out)  */
/*   window[b,v,:] <- shift left, append xBC[b,v]      (conv_state, in place)  */
/*   xBC' = silu(sum_k window[b,v,k] conv_w[v,k] + conv_b[v])                  */
/*   dt   = clamp(softplus(dt_raw + dt_bias), dt_min, dt_max) ; dA = exp(dt A)  */
/*   h[b,h,p,n] <- h dA + (dt B[g,n]) x[h,p]          (ssm_state, in place)    */
/*   y = sum_n h C[g,n] + D x ; out = RmsNormGated(y, z)                       */
/*                                                                             */
/* conv_dim = d_inner + 2 ngroups dstate, d_inner = nheads headdim; head h     */
/* reads group h / (nheads / ngroups).  RmsNormGated (norm/rms_norm_gated.rs:  */
/* 70-135): norm_before_gate = 0 gives g = y silu(z), out = g / sqrt(mean(g^2) */
/* + eps) w; 1 gives out = y / sqrt(mean(y^2) + eps) w silu(z); the mean runs  */
/* over all d_inner channels of a row.  The caches keep the reference's        */
/* Mamba2Cache layout (src/mamba2/cache.rs:98-122): conv_bvk [b, conv_dim, K]   */
/* and ssm_bhpr [b, nheads, headdim, dstate], both f32 and contiguous.         */
/* ------------------------------------------------------------------------- */
typedef struct mamba2_step_args {
    int32_t batch, nheads, headdim, ngroups, dstate, conv_kernel;
    int32_t zxbcdt_dtype;             /* mamba_dtype of zxbcdt                  */
    int32_t out_dtype;                /* mamba_dtype of out                     */
    int32_t norm_before_gate;         /* 0 (reference default) or 1             */
    const void* zxbcdt; int64_t zxbcdt_sb;  /* [b, d_inner + conv_dim + nheads] */
    float* conv_state;                /* [b, conv_dim, conv_kernel], in/out     */
    const float* conv_w;              /* [conv_dim, conv_kernel] (Conv1d [v,1,k]) */
    const float* conv_b;              /* [conv_dim] or NULL                      */
    const float* dt_bias;             /* [nheads] or NULL                        */
    const float* A;                   /* [nheads], A = -exp(a_log)               */
    const float* D;                   /* [nheads] or NULL (= 0)                  */
    float dt_min, dt_max;             /* dt_limit (reference default 0, 65504)  */
    const float* norm_w;              /* [d_inner] gated-RMSNorm gamma           */
    float* ssm_state;                 /* [b, nheads, headdim, dstate], in/out   */
    void* out; int64_t out_sb;        /* [b, d_inner]                            */
} mamba2_step_args;

size_t mamba2_step_workspace_size(const mamba2_step_args* args);
/* Replaces Mamba2::step (src/mamba2/mamba2.rs:820-1004) from the in_proj      */
/* split (:849-861) to the gated norm (:995); in_proj/out_proj stay dense      */
/* products the caller runs.                                                   */
int mamba2_step_ssm(const mamba2_step_args* args, void* workspace, size_t workspace_bytes,
                    mamba_stream_t stream);
/* As mamba2_step_ssm, recording the caller's HIP events around the state-     */
/* update kernel (benchmark timing; no counterpart in the reference).          */
int mamba2_step_ssm_timed(const mamba2_step_args* args, void* workspace, size_t workspace_bytes,
                          mamba_stream_t stream, void* event_start, void* event_stop);

/* ------------------------------------------------------------------------- */
/* Dense-product weight packing for the fused decode entry points.            */
/* A Burn Linear weight [d_in, d_out] (row-major, leading dimension ld, f32 or */
/* bf16) is repacked once, at model load, into bf16 tiles in MFMA operand      */
/* order; d_in must be a multiple of 16.  mamba_linear_packed_size returns the */
/* bytes of the packed copy (0 for unsupported shapes).  No counterpart in the */
/* reference (Burn multiplies its stored layout directly).                     */
/* ------------------------------------------------------------------------- */
size_t mamba_linear_packed_size(int32_t d_in, int32_t d_out);
int mamba_linear_pack(const void* weight, int32_t d_in, int32_t d_out, int64_t ld, int32_t dtype,
                      void* packed, mamba_stream_t stream);

/* y[r, :] = x[r, :] W (+ bias) for 1 <= rows <= 256 (one token per sequence), */
/* W packed by mamba_linear_pack: burn::nn::Linear::forward as the decode      */
/* steps use it (in_proj/x_proj/dt_proj/out_proj, src/mamba1/mamba1.rs:551,    */
/* 633-644,609; src/mamba2/mamba2.rs:850,1000).  bf16 operands, f32            */
/* accumulation.  A bf16 x with 16-byte aligned rows (x_ld a multiple of 8) is */
/* read in place; any other x is repacked into the workspace first.  The       */
/* workspace also holds k-split partial sums for large weights; its size may   */
/* be 0 (then workspace may be NULL).                                          */
typedef struct mamba_linear_args {
    int32_t rows, d_in, d_out;
    int32_t x_dtype, y_dtype;         /* mamba_dtype                            */
    const void* x; int64_t x_ld;      /* [rows, d_in]                           */
    const void* packed_w;             /* mamba_linear_pack output               */
    const float* bias;                /* [d_out] or NULL                        */
    void* y; int64_t y_ld;            /* [rows, d_out]                          */
} mamba_linear_args;

size_t mamba_linear_workspace_size(const mamba_linear_args* args);
int mamba_linear_fwd(const mamba_linear_args* args, void* workspace, size_t workspace_bytes,
                     mamba_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Fused pre-norm Mamba-2 layer decode step (Layer::step_one around           */
/* Mamba2::step, src/modules/layer.rs:224-232 + src/mamba2/mamba2.rs:820-1004): */
/*                                                                             */
/*   x += out_proj(RmsNormGated(ssm_step(in_proj(RmsNorm(x)))))                */
/*                                                                             */
/* with the same state update as mamba2_step_ssm and the caches updated in     */
/* place.  in_proj / out_proj are the packed weights of mamba_linear_pack.     */
/* Kernels: RmsNorm into the product's operand layout, in_proj (k-split f32    */
/* partial planes), the state update (sums the in_proj planes, writes the      */
/* out_proj operand g * norm_w), out_proj (planes), and a per-row pass that    */
/* sums those planes, applies the gated norm's 1/rms (a per-row scalar, so it  */
/* commutes with the product), the bias and the residual add, and slides the  */
/* B/C conv windows.  The projections stay in f32 (zxbcdt_dtype is ignored).  */
/* Supports headdim 64, dstate 64 or 128, conv_kernel 4, batch <= 256,         */
/* d_model % 16 == 0 and <= 4096; other shapes return MAMBA_ERR_UNSUPPORTED    */
/* (use mamba2_step_ssm with a separate product).  x, the packed weights,      */
/* pre_norm_w, out_proj_b and the caches must be 16-byte aligned.              */
/* ------------------------------------------------------------------------- */
typedef struct mamba2_layer_args {
    int32_t batch, d_model, nheads, headdim, ngroups, dstate, conv_kernel;
    int32_t norm_before_gate;
    int32_t zxbcdt_dtype;             /* precision of the in_proj result (bf16 like a bf16 model) */
    float* x; int64_t x_sb;           /* [b, d_model] f32 residual stream, in/out */
    const float* pre_norm_w;          /* [d_model] RmsNorm gamma of the layer   */
    const void* in_proj;              /* packed [d_model, d_in_proj]            */
    const float* in_proj_b;           /* [d_in_proj] or NULL                    */
    const void* out_proj;             /* packed [d_inner, d_model]              */
    const float* out_proj_b;          /* [d_model] or NULL                      */
    float* conv_state;                /* [b, conv_dim, conv_kernel], in/out     */
    const float* conv_w;              /* [conv_dim, conv_kernel]                */
    const float* conv_b;              /* [conv_dim] or NULL                     */
    const float* dt_bias;             /* [nheads] or NULL                       */
    const float* A;                   /* [nheads]                               */
    const float* D;                   /* [nheads] or NULL                       */
    float dt_min, dt_max;
    const float* norm_w;              /* [d_inner] gated-RMSNorm gamma          */
    float* ssm_state;                 /* [b, nheads, headdim, dstate], in/out   */
    int32_t concurrent;               /* 1: another stream runs other rows' layers */
                                      /* beside this call (a batch split over two */
                                      /* streams); with at most 32 rows the products */
                                      /* then stream in fewer, wider workgroups,  */
                                      /* which run faster beside a state kernel.  */
                                      /* Results do not depend on it.  0 otherwise. */
} mamba2_layer_args;

size_t mamba2_layer_workspace_size(const mamba2_layer_args* args);
int mamba2_layer_step(const mamba2_layer_args* args, void* workspace, size_t workspace_bytes,
                      mamba_stream_t stream);
/* As mamba2_layer_step, recording the caller's HIP events around the state-  */
/* update kernel (benchmark timing; no counterpart in the reference).          */
int mamba2_layer_step_timed(const mamba2_layer_args* args, void* workspace, size_t workspace_bytes,
                            mamba_stream_t stream, void* event_start, void* event_stop);

/* n_layers pre-norm layers on one residual stream, one token per sequence:    */
/* the decode side of Layers::step without class latents                       */
/* (src/modules/layers.rs:427-…).  Every layer shares the shapes and x; the    */
/* residual pass of layer l also writes the normed operand of layer l + 1, so  */
/* a layer is four kernels.  Workspace: mamba2_layer_workspace_size of any one */
/* layer.  The _timed variant records event_start[l] / event_stop[l] around    */
/* layer l's state-update kernel (benchmark timing).                           */
int mamba2_stack_step(const mamba2_layer_args* layers, int32_t n_layers, void* workspace,
                      size_t workspace_bytes, mamba_stream_t stream);
int mamba2_stack_step_timed(const mamba2_layer_args* layers, int32_t n_layers, void* workspace,
                            size_t workspace_bytes, mamba_stream_t stream, void* const* event_start,
                            void* const* event_stop);

/* mamba2_stack_step without a workspace argument and without any allocation: */
/* no counterpart in the reference.  It is for callers that cannot allocate    */
/* device memory (code under HIP graph capture, tight serving loops, harnesses */
/* that forbid hipMalloc).  The workspace is a file-scope device array of      */
/* MAMBA2_STACK_NOALLOC_SCRATCH_BYTES, one per GPU, held until the process     */
/* ends; a stack whose mamba2_layer_workspace_size exceeds it is rejected with */
/* MAMBA_ERR_WORKSPACE before any launch.  48 MiB holds every one-group stack  */
/* mamba2_stack_step accepts at expand 2 (batch <= 256, d_model <= 4096; the   */
/* 2.7B-shaped stack needs 29.5 MiB at batch 256).  Nothing in it needs to     */
/* start at zero.  Every call on a GPU shares that GPU's array, so calls that  */
/* overlap on one GPU (other streams or host threads) race; serialise them.    */
#define MAMBA2_STACK_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)
int mamba2_stack_step_noalloc(const mamba2_layer_args* layers, int32_t n_layers, mamba_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Residual add + RmsNorm over rows (src/modules/norm/rms_norm.rs:53-98), the  */
/* pre-norm and residual of Layer::step_one (src/modules/layer.rs:224-232):    */
/*   x[r,:] += add[r,:]                      (when add != NULL; x is f32)     */
/*   out[r,:] = x[r,:] / sqrt(mean(x[r,:]^2) + eps) * weight   (when out)     */
/* ------------------------------------------------------------------------- */
typedef struct mamba_rmsnorm_args {
    int32_t rows, cols;
    int32_t add_dtype, out_dtype;     /* mamba_dtype of add and out             */
    float* x;         int64_t x_sr;   /* [rows, cols] f32, updated when add     */
    const void* add;  int64_t add_sr; /* [rows, cols] or NULL                    */
    const float* weight;              /* [cols]; required when out != NULL       */
    void* out;        int64_t out_sr; /* [rows, cols] or NULL                    */
} mamba_rmsnorm_args;

int mamba_rmsnorm(const mamba_rmsnorm_args* args, mamba_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Mamba-2 prefill prologue: Mamba2::forward steps 2 and 4                     */
/* (src/mamba2/mamba2.rs:618-699).  From the in_proj rows [b, l, row]:         */
/*   xbc[b,l,c] = silu(conv_b[c] + sum_k conv_w[c,k] xpad[b,c,l+k])            */
/* with xpad = [conv_state[b,c,1:] | proj[b,:,xbc_offset + c]] (causal, valid), */
/*   dt[b,l,h] = clamp(softplus(proj[b,l,dt_offset + h] + dt_bias[h]),         */
/*                     dt_min, dt_max),                                         */
/* then conv_state[b,c,:] = the last `kernel` columns of xpad (:652-655),      */
/* updated in place after the outputs are computed.  nheads = 0 skips dt      */
/* (dt_bias and dt may then be NULL): the Mamba-1 prefill conv, layer 2 of    */
/* Mamba1::forward (src/mamba1/mamba1.rs:300-340), over the x half of the     */
/* in_proj rows.                                                               */
/* ------------------------------------------------------------------------- */
typedef struct mamba2_conv_args {
    int32_t batch, seqlen, channels, kernel, nheads; /* channels = conv_dim; kernel <= 8; nheads >= 0 */
    int32_t in_dtype, out_dtype;                     /* proj; xbc                  */
    const void* proj;   int64_t proj_sb, proj_sl;    /* [b, l, row]                */
    int32_t xbc_offset, dt_offset;                   /* column offsets in a row    */
    const float* conv_w;                             /* [channels, kernel]         */
    const float* conv_b;                             /* [channels] or NULL         */
    float* conv_state;                               /* [b, channels, kernel] in/out */
    const float* dt_bias;                            /* [nheads]                   */
    float dt_min, dt_max;
    void* xbc;          int64_t xbc_sb, xbc_sl;      /* [b, l, channels] out       */
    float* dt;                                       /* [b, l, nheads] out         */
} mamba2_conv_args;

int mamba2_conv_fwd(const mamba2_conv_args* args, mamba_stream_t stream);

/* Gated RMSNorm over rows of `width` (RmsNormGated::forward,                  */
/* src/modules/norm/rms_norm_gated.rs:70-135; Mamba2::forward step 7,         */
/* src/mamba2/mamba2.rs:776):                                                  */
/*   norm_before_gate == 0:  g = y silu(z);  out = g / sqrt(mean(g^2) + eps) gamma */
/*   norm_before_gate != 0:  out = y / sqrt(mean(y^2) + eps) gamma silu(z)    */
/* eps is the reference's div_eps of its dtype (src/utils/mod.rs:50-95).       */
typedef struct mamba2_gated_norm_args {
    int32_t batch, seqlen, width, norm_before_gate;
    int32_t y_dtype, z_dtype, out_dtype;
    float eps;
    const void* y;      int64_t y_sb, y_sl;          /* [b, l, width]              */
    const void* z;      int64_t z_sb, z_sl;          /* [b, l, width]              */
    const float* gamma;                              /* [width]                    */
    void* out;          int64_t out_sb, out_sl;      /* [b, l, width]              */
} mamba2_gated_norm_args;

int mamba2_gated_rmsnorm(const mamba2_gated_norm_args* args, mamba_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA_HIP_H */
