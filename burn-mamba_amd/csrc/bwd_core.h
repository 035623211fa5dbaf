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

// Sum of 16 per-lane values over the 32 lanes of a wave half, scattered: lane
// i32 returns the total of value (i32 >> 1) (both lanes of a pair hold it).
__device__ __forceinline__ float bwd_half_sum16(const float (&v)[16], int i32) {
    float w[8], x[4], y[2];
    const bool b4 = (i32 >> 4) & 1, b3 = (i32 >> 3) & 1, b2 = (i32 >> 2) & 1, b1 = (i32 >> 1) & 1;
#pragma unroll
    for (int q = 0; q < 8; ++q) w[q] = (b4 ? v[8 + q] : v[q]) + __shfl_xor(b4 ? v[q] : v[8 + q], 16, 64);
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = (b3 ? w[4 + q] : w[q]) + __shfl_xor(b3 ? w[q] : w[4 + q], 8, 64);
#pragma unroll
    for (int q = 0; q < 2; ++q) y[q] = (b2 ? x[2 + q] : x[q]) + __shfl_xor(b2 ? x[q] : x[2 + q], 4, 64);
    float z = (b1 ? y[1] : y[0]) + __shfl_xor(b1 ? y[0] : y[1], 2, 64);
    return z + __shfl_xor(z, 1, 64);
}
// Sum over the 32 lanes of a wave half (every lane of the half gets it).
__device__ __forceinline__ float bwd_half_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ void bwd_put4(float* dst, float4 v) {
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
}

}  // namespace mamba
