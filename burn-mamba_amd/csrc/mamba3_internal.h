// Mamba-3 prefill internals shared by the prologue kernels and the fused
// prologue + SSD kernel: the prologue's parameter block, the coefficient
// functions and the lane-exchange helpers.
#pragma once

#include "common.h"

namespace mamba {

struct M3PrepParams {
    int nb, L, H, P, G, N, M, R, A;
    bool proj_bf16, io_bf16;
    const void* proj; int64_t proj_sb, proj_sl;
    const float* ssm; float* kst; float* vst; const float* ang; float* ang_out;
    const float* dt_bias; float a_floor, dt_lo, dt_hi, span;
    const float* bnw; const float* cnw; const float* bbias; const float* cbias; const float* mx;
    void* v; void* Bo; void* Co;
    float* da; float* gm; float* sc;
    float* h0;
};

// ---- the prologue's arithmetic, shared by every Mamba-3 prefill kernel.
// The segment-parallel prep (mamba3_prep.hip) and the prologue fused into the
// scan (mamba3_fused.hip) form the same coefficients, angles and B / C rows
// from the same in_proj row with these functions, bit for bit: the fused
// kernel then equals the prep followed by the seam scan exactly.  Hardware
// exp / reciprocal / rsqrt / sin / cos (a few ulp; the library's correctly
// rounded forms measured 50 % slower in the fused kernel and moved no B / C
// element closer to the f64 oracle: the f32 angle recurrence sets that
// distance) and explicit fmas (no contraction choice left to the compiler).

__device__ __forceinline__ float m3p_softplus(float x) { return x > 18.f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float m3_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// tanh from one exponential: sign(x) (1 - e) / (1 + e), e = exp(-2 |x|) <= 1
__device__ __forceinline__ float m3_tanh(float x) {
    const float e = __expf(-2.f * fabsf(x));
    return copysignf((1.f - e) * __builtin_amdgcn_rcpf(1.f + e), x);
}
// cos and sin of an angle in [-pi, pi]
__device__ __forceinline__ void m3_cossin(float a, float& c, float& s) {
    c = __cosf(a);
    s = __sinf(a);
}
// dt, da = dt A, lambda of one (position, head) from its raw dd_dt, dd_A, lambda columns
// (trapezoidal_coefficients, helpers.rs:42-73)
__device__ __forceinline__ void m3_coef(float raw_dt, float raw_da, float raw_lam, float dt_bias, float a_floor,
                                        float dt_lo, float dt_hi, float& dt, float& da, float& lam) {
    dt = fminf(fmaxf(m3p_softplus(raw_dt + dt_bias), dt_lo), dt_hi);
    da = dt * -fmaxf(m3p_softplus(raw_da), a_floor);
    lam = m3_sigmoid(raw_lam);
}
// angle increment dt range pi tanh(rot) (rotation/mod.rs:653-679)
__device__ __forceinline__ float m3_angle_inc(float dt, float raw_rot, float span) {
    return dt * (m3_tanh(raw_rot) * span);
}

// Cumulative angles in fixed point: multiples of 2^-24 rad in an int32,
// reduced modulo Q2PI (2 pi in those units, odd) to the canonical range
// [-(Q2PI - 1) / 2, (Q2PI - 1) / 2].  Integer sums do not depend on their
// association, so every kernel (whatever its segmentation of the sequence)
// gets the same angle at every position: the cache's angle plus the sum of
// the increments before it, each put on the 6e-8 rad grid (the reference's
// f32 cumsum drifts by far more over long sequences).  Every value added is
// canonical, and sums of at most 16 of them stay below 2^31.
constexpr float kAngUnit = 16777216.f;           // units per radian (2^24)
constexpr int kQ2Pi = 105414357;                 // rint(2 pi 2^24) - 1, odd
constexpr float kInvQ2Pi = 1.f / 105414357.f;
__device__ __forceinline__ int m3_ang_reduce(int q) {
    // the quotient's estimate may be off by one: the two corrections make the
    // result exact and canonical
    q -= (int)rintf((float)q * kInvQ2Pi) * kQ2Pi;
    if (q > kQ2Pi / 2) q -= kQ2Pi;
    if (q < -(kQ2Pi / 2)) q += kQ2Pi;
    return q;
}
// an angle in radians (a cache angle or one increment) onto the grid: first
// reduced to [-pi, pi] in f32 (so that its grid value fits an int32), then its
// whole radians and its fraction (exact in f32) scaled separately, so that the
// fraction keeps the grid's full resolution
__device__ __forceinline__ int m3_ang_fix(float a) {
    constexpr float two_pi = 6.28318530717958647692f;
    const float r = __builtin_fmaf(-rintf(a * (1.f / two_pi)), two_pi, a);  // explicit: no contraction choice
    const float w = rintf(r);
    return m3_ang_reduce((int)w * (int)kAngUnit + (int)rintf((r - w) * kAngUnit));
}
// a canonical grid angle as f32 radians in [-pi, pi]
__device__ __forceinline__ float m3_ang_rad(int q) { return (float)q * (1.f / kAngUnit); }

// One B / C row piece of 8 columns: the sum of squares (to be completed over
// the row's lanes), the norm weight and bias, the rotation
// y' = c y + s y_partner (s carries the pair's sign).
__device__ __forceinline__ float m3_sumsq8(const float* y) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(y[e], y[e], ss);
    return ss;
}
__device__ __forceinline__ float m3_rms_inv(float ss, int n) {
    return __builtin_amdgcn_rsqf(ss / (float)n + kDivEpsF32);  // the argument is >= eps: a normal number
}
__device__ __forceinline__ float m3_norm(float y, float rms, float w, float bias) {
    return __builtin_fmaf(y * rms, w, bias);
}
__device__ __forceinline__ float m3_rot(float c, float y, float s, float o) { return __builtin_fmaf(c, y, s * o); }
// Lane exchanges inside aligned groups of a wave, without LDS addressing:
// DPP for the quad and 16-lane-row patterns, ds_swizzle (bit-mask mode) for
// the other xor distances below 32.
template <int CTRL>
__device__ __forceinline__ float m3_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <int K>
__device__ __forceinline__ float m3_xor(float x) {  // value of lane (lane ^ K), K < 32
    if constexpr (K == 1) return m3_dpp<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    else if constexpr (K == 2) return m3_dpp<0x4E>(x);  // quad_perm [2, 3, 0, 1]
    else if constexpr (K == 8) return m3_dpp<0x128>(x);  // row_ror:8 (lane ^ 8 inside a 16-lane row)
    else return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1F | (K << 10)));
}
// sum over an aligned group of G lanes (G a power of two <= 32), in every lane
template <int G>
__device__ __forceinline__ float m3_group_sum(float x) {
    if constexpr (G >= 32) x += m3_xor<16>(x);
    if constexpr (G >= 16) x += m3_dpp<0x140>(x);  // row_mirror: i <-> 15 - i
    if constexpr (G >= 8) x += m3_dpp<0x141>(x);   // row_half_mirror: i <-> 7 - i (per 8)
    if constexpr (G >= 4) x += m3_dpp<0x1B>(x);    // quad_perm [3, 2, 1, 0]
    if constexpr (G >= 2) x += m3_dpp<0xB1>(x);    // quad_perm [1, 0, 3, 2]
    return x;
}


// Host side (mamba3_prep.hip): the prologue's parameter block from the C-ABI
// arguments (with need_outputs = false the v / B / C / da / gamma / scale
// outputs may be NULL), and the launch of the beta-seed kernel that writes
// the initial state p.h0 from p.ssm and the cache tail.
int m3_prep_params(const mamba3_prep_args* a, M3PrepParams* out, bool need_outputs);
void m3_launch_seed(const M3PrepParams& p, hipStream_t s);

}  // namespace mamba
