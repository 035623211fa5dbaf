// f32 MFMA helpers shared by the SSD backward kernels (ssd2_bwd.hip,
// ssd3_bwd.hip): v_mfma_f32_32x32x2_f32 (f32 operands and accumulation).  For
// that instruction lane l supplies A[l % 32][k0 + l / 32] and
// B[k0 + l / 32][l % 32], and accumulator r of lane l holds
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].  LDS rows are padded to an odd
// number of words, so that both the K-major reads (32 rows, one column) and
// the row-major reads (32 consecutive words) of a half-wave fall in 32
// distinct banks.
#pragma once

#include <hip/hip_runtime.h>

namespace mamba {

typedef float bwd_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kFP = 64, kFN = 128;                 // headdim, dstate of the MFMA paths
constexpr int kSX = 65, kSB = 129, kSQ = 33;       // padded row lengths (words)

__device__ __forceinline__ bwd_f32x16 bwd_mfma(float a, float b, bwd_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
// the accumulator row of register r for a lane in wave half hf
__device__ __forceinline__ int bwd_row(int r, int hf) { return 8 * (r >> 2) + 4 * hf + (r & 3); }

// Lane exchanges inside 16-lane rows on DPP moves (no LDS round trip): xor 1
// and xor 2 are quad permutations, xor 8 the row rotation by 8, and xor 4 the
// quad reversal (xor 3) followed by the half-row mirror (xor 7).  Exchanges
// across rows (xor 16) go through the LDS permute.
template <int CTRL>
__device__ __forceinline__ float bwd_dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float bwd_xor1(float v) { return bwd_dpp_mov<0xb1>(v); }   // quad_perm [1,0,3,2]
__device__ __forceinline__ float bwd_xor2(float v) { return bwd_dpp_mov<0x4e>(v); }   // quad_perm [2,3,0,1]
__device__ __forceinline__ float bwd_xor4(float v) {                                   // row_half_mirror o quad_perm [3,2,1,0]
    return bwd_dpp_mov<0x141>(bwd_dpp_mov<0x1b>(v));
}
__device__ __forceinline__ float bwd_xor8(float v) { return bwd_dpp_mov<0x128>(v); }  // row_ror:8

// Sum of 16 per-lane values over the 32 lanes of a wave half, scattered: lane
// i32 returns the total of value (i32 >> 1) (both lanes of a pair hold it).
__device__ __forceinline__ float bwd_half_sum16(const float (&v)[16], int i32) {
    float w[8], x[4], y[2];
    const bool b4 = (i32 >> 4) & 1, b3 = (i32 >> 3) & 1, b2 = (i32 >> 2) & 1, b1 = (i32 >> 1) & 1;
#pragma unroll
    for (int q = 0; q < 8; ++q) w[q] = (b4 ? v[8 + q] : v[q]) + __shfl_xor(b4 ? v[q] : v[8 + q], 16, 64);
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = (b3 ? w[4 + q] : w[q]) + bwd_xor8(b3 ? w[q] : w[4 + q]);
#pragma unroll
    for (int q = 0; q < 2; ++q) y[q] = (b2 ? x[2 + q] : x[q]) + bwd_xor4(b2 ? x[q] : x[2 + q]);
    const float z = (b1 ? y[1] : y[0]) + bwd_xor2(b1 ? y[0] : y[1]);
    return z + bwd_xor1(z);
}
// Sum over the 32 lanes of a wave half (every lane of the half gets it).
__device__ __forceinline__ float bwd_half_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    v += bwd_xor8(v);
    v += bwd_xor4(v);
    v += bwd_xor2(v);
    return v + bwd_xor1(v);
}

__device__ __forceinline__ void bwd_put4(float* dst, float4 v) {
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
}

}  // namespace mamba
