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

__device__ __forceinline__ float m3p_softplus(float x) { return x > 18.f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float m3p_wrap(float a) {
    const float two_pi = 6.28318530717958647692f;
    return a - rintf(a * (1.f / two_pi)) * two_pi;
}
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

// tanh from one exponential: sign(x) (1 - e) / (1 + e), e = exp(-2 |x|) <= 1
__device__ __forceinline__ float m3_tanh(float x) {
    const float e = __expf(-2.f * fabsf(x));
    return copysignf((1.f - e) / (1.f + e), x);
}

// Host side (mamba3_prep.hip): the prologue's parameter block from the C-ABI
// arguments (with need_outputs = false the v / B / C / da / gamma / scale
// outputs may be NULL), and the launch of the beta-seed kernel that writes
// the initial state p.h0 from p.ssm and the cache tail.
int m3_prep_params(const mamba3_prep_args* a, M3PrepParams* out, bool need_outputs);
void m3_launch_seed(const M3PrepParams& p, hipStream_t s);

}  // namespace mamba
