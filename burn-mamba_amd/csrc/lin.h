// Weight-streaming dense product for one-token-per-sequence steps (decode),
// shared by the step entry points.
#pragma once

#include "common.h"

namespace mamba {

typedef __bf16 lin_bf16x8_t __attribute__((ext_vector_type(8)));

// Packed operand formats (v_mfma_f32_32x32x16_bf16, lane l, r = l % 32, half = l / 32):
//   weight W[k][n] (K x N):  block (j, s) = 32 columns x 16 k, lane l holds
//                            W[16 s + 8 half + e][32 j + r], e = 0..7 (16 bytes);
//                            blocks ordered j-major: offset (j * KS + s) * 64 lanes.
//   activation A[m][k] (M x K): block (s, i) = 32 rows x 16 k, lane l holds
//                            A[32 i + r][16 s + 8 half + e];
//                            blocks ordered s-major: offset (s * MT + i) * 64 lanes.
// KS = K / 16; MT = lin_mt(M), the number of 32-row tiles rounded up to 1, 2, 4
// or 8 (the kernel is instantiated for those).  Rows m >= M of an activation
// block are never written and never reach an output (row m of the product
// depends on row m of A only).
inline int lin_mt(int M) { return M <= 32 ? 1 : M <= 64 ? 2 : M <= 128 ? 4 : 8; }
inline size_t lin_weight_elems(int K, int N) { return (size_t)((N + 31) / 32) * 32 * K; }
inline size_t lin_act_elems(int M, int K) { return (size_t)lin_mt(M) * 32 * K; }

__device__ __forceinline__ int64_t lin_act_offset(int m, int k, int MT) {
    const int s = k >> 4, i = m >> 5, lane = (m & 31) + 32 * ((k >> 3) & 1);
    return ((int64_t)(s * MT + i) * 64 + lane) * 8 + (k & 7);
}

enum LinEpilogue { LIN_STORE = 0, LIN_PARTIAL = 1 };

struct LinParams {
    int M, N, K, MT;         // MT = lin_mt(M)
    int S;                   // k-splits across workgroups (grid.y)
    const lin_bf16x8_t* W;   // packed weight
    const lin_bf16x8_t* A;   // packed activation, or NULL when X is given
    // row-major bf16 activation [M][x_ld] read in place (16-byte aligned rows):
    // lane l of block (s, i) holds 8 consecutive k of one row, 16 contiguous
    // bytes, so no packing pass is needed
    const bf16_t* X; int64_t x_ld;
    int NW;                  // waves per workgroup (0: the default for MT)
    // column parts per 32-column tile (0 or 1: one; 2 or 4): CS workgroups
    // share a tile, each loading only its 32 / CS columns' lanes of every
    // weight block (the other lanes read zero) and storing only its columns,
    // so a product with few column tiles streams from CS times the
    // workgroups without a summing pass
    int CS;
    // LIN_STORE (S == 1): out[m, n] = acc + bias
    const float* bias;       // [N] or NULL
    void* out; int64_t out_ld; bool out_bf16;
    // LIN_PARTIAL: part[z][m][n] = acc over k-split z (f32, planes of M x N);
    // the consumer sums the S planes in a fixed order
    float* part;
};

// k-splits for a product: enough workgroups (~1300 of 4 waves, ~10 weight
// blocks per wave) to stream the weight at full HBM rate, fewer for large M
// where the partial planes grow.
#ifndef MAMBA_LIN_MAXS_MID
#define MAMBA_LIN_MAXS_MID 2   // k-split cap for 32 < M <= 64 (fewer partial planes)
#endif
#ifndef MAMBA_LIN_PART_BYTES
#define MAMBA_LIN_PART_BYTES (6 << 20)  // partial planes small enough to split further
#endif
inline int lin_splits(int M, int K, int N) {
    const int ks = K / 16, tiles = (N + 31) / 32;
    const int cap = M <= 32 ? 16 : M <= 64 ? MAMBA_LIN_MAXS_MID : 2;
    auto more = [&](int s) { return ks / (2 * s) >= 40 && tiles * s < 1024; };
    int s = 1;
    while (s < cap && more(s)) s *= 2;
    // products with few column tiles (out_proj: N = d_model) have small
    // planes: keep splitting while they stay small, so that enough workgroups
    // stream the weight
    while (s < 16 && more(s) && (size_t)2 * s * M * N * 4 <= (size_t)MAMBA_LIN_PART_BYTES) s *= 2;
    return s;
}
inline size_t lin_part_elems(int M, int N, int S) { return (size_t)S * M * N; }

// Launch the product on `stream`; the caller has validated the shapes
// (K % 16 == 0, 1 <= M <= 256).
void lin_launch(const LinParams& p, int epilogue, hipStream_t stream);

}  // namespace mamba
