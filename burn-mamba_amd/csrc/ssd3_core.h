// Shared pieces of the Mamba-3 single-SSD MFMA scans (bf16 operands, f32
// accumulators, headdim 64 in two 32-wide halves, dstate 128, 128 fused
// positions per chunk): the MFMA helpers, the per-workgroup LDS layout, and
// the y tile and the state update of one wave.  Included by the SSD-seam
// kernel and by the fused prologue + SSD kernel.
#pragma once

#include "common.h"

namespace mamba {

typedef __bf16 s3_bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 s3_bf16x4_t __attribute__((ext_vector_type(4)));
typedef float s3_f32x16_t __attribute__((ext_vector_type(16)));

constexpr float kLog2eS3 = 1.4426950408889634f;

__device__ __forceinline__ s3_f32x16_t s3_mfma(s3_bf16x8_t a, s3_bf16x8_t b, s3_f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ s3_f32x16_t s3_zero() {
    s3_f32x16_t z;
#pragma unroll
    for (int v = 0; v < 16; ++v) z[v] = 0.f;
    return z;
}

// Raw buffer access (gfx9 descriptor word 3): offsets at or past `bytes`
// read as zero and drop on store, which clips chunks at the sequence end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t s3_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 s3_bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float s3_bld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ float s3_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float s3_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two-term bf16 operands.  The inputs (v, B, C) are bf16, but three operands
// of the scan are formed inside it in f32: the state entering a chunk (the A
// operand of C.h), the decay-weighted C.B^T (the B operand of v^T.M) and the
// weighted v^T of the state update.  Each is carried as hi + lo, two bf16
// values with hi = bf16(x) and lo = bf16(x - hi) (about 16 significant bits),
// and enters its product as two MFMAs, so that the products are exact to
// ~2^-17 relative instead of bf16's 2^-9: with QK-normed B / C (|C.B| ~ N) a
// single bf16 rounding of these operands moves outputs near zero by more than
// 1e-2.
__device__ __forceinline__ __bf16 s3_h16(float x) { return (__bf16)x; }
__device__ __forceinline__ __bf16 s3_l16(float x) { return (__bf16)(x - (float)(__bf16)x); }
// hi + lo of a product a b: hi = bf16(a b), and the residual a b - hi formed
// by an explicit fma (exact before its rounding), so that no kernel's result
// depends on whether the compiler contracts a b - hi into an fma: the kernels
// that must agree bit for bit (the fused Mamba-3 prefill and the seam scan)
// split their products this way.
__device__ __forceinline__ float s3_res(float a, float b, float hi) { return __builtin_fmaf(a, b, -hi); }
__device__ __forceinline__ void s3_split(float a, float b, __bf16& hi, __bf16& lo) {
    hi = (__bf16)(a * b);
    lo = (__bf16)s3_res(a, b, (float)hi);
}

// LDS of one workgroup (about 109 KB at QF = 128 with HB = 2).  HB: buffers
// of the chunk-entry state (2: the next chunk's state is written while this
// chunk's is read; 1: the writer waits for the next chunk).  NY: y tiles
// staged for the store (one per wave; a caller that stores y straight from
// its accumulators keeps one unused tile).
template <int QF, int HB = 2, int NY = 4>
struct __align__(16) Ssd3Lds {
    bf16_t xT[32][QF + 8];      // v^T of the chunk (headdim half x positions)
    bf16_t xTw[32][QF + 8];     // w_j v^T[p][j], the state GEMM's A operand (hi part)
    bf16_t xTwl[32][QF + 8];    // its lo part
    bf16_t B[QF][136];          // B rows of the chunk (positions x dstate)
    bf16_t h[HB][32][136];      // state entering the chunk (MFMA operand, hi part)
    bf16_t hl[HB][32][136];     // its lo part
    bf16_t y[NY][32][40];       // per-wave y tile staging
    float cs2[QF];              // within-chunk cumulative da, log2 units
    float sc[QF], gm[QF];       // scale and gamma per position
    float st[QF];               // step index of each position (read per chunk: keeps the
                                // diagonal masks in the loop rather than hoisted to SGPRs)
    float w[QF];                // scale_j exp(cs_end - cs_j)
    float f[QF / 32 - 1][QF];   // scale_j exp(cs_r0 - cs_j) for tile starts r0 = 32, 64, ..
    float red[4], anc[QF / 32];
};

// y of output tile IT (positions 32 IT .. 32 IT + 31 of the chunk) for this
// wave's headdim half, in one accumulator (lane = column i, so the per-i
// factors are per-lane scalars applied between the MFMA chains):
//   y  = C_i.h_in;  y *= exp(cs_r0);  y += lower tiles (f_IT[j]);
//   y *= exp(cs_i - cs_r0);  y += diagonal tile (exact per-(j, i) factor)
// LEAN: a scheduling barrier between the lower-tile blocks, so that the
// compiler does not hoist every block's LDS operands at once (for callers
// that run two waves per SIMD within 256 registers).
template <int QF, int IT, bool LEAN = false, int HB, int NY>
__device__ __forceinline__ void ssd3_y_tile(Ssd3Lds<QF, HB, NY>& S, const s3_bf16x8_t (&cfr)[8], int cur, int r, int half,
                                            s3_f32x16_t& y) {
    constexpr int NK = 8;
    const int il = IT * 32 + r;
    const float cs_i = S.cs2[il];
    const float cs_r0 = S.cs2[IT * 32];
    const float gm_i = S.gm[il];
    const float ti = S.st[il];  // chunks and tiles start on step boundaries
    y = s3_zero();
#pragma unroll
    for (int kn = 0; kn < NK; ++kn) {
        y = s3_mfma(*(const s3_bf16x8_t*)&S.h[cur][r][kn * 16 + 8 * half], cfr[kn], y);
        y = s3_mfma(*(const s3_bf16x8_t*)&S.hl[cur][r][kn * 16 + 8 * half], cfr[kn], y);
    }
    {
        const float e0 = __builtin_amdgcn_exp2f(cs_r0);
#pragma unroll
        for (int v = 0; v < 16; ++v) y[v] *= e0;
    }
#pragma unroll
    for (int jt = 0; jt <= IT; ++jt) {
        if constexpr (LEAN) __builtin_amdgcn_sched_barrier(0);
        s3_f32x16_t d = s3_zero();
#pragma unroll
        for (int kn = 0; kn < NK; ++kn)
            d = s3_mfma(*(const s3_bf16x8_t*)&S.B[jt * 32 + r][kn * 16 + 8 * half], cfr[kn], d);
        // d[v] = C_i . B_j for j = 32 jt + 8 (v / 4) + 4 half + v % 4
        float fac[16];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
            const int j0 = jt * 32 + 8 * gq + 4 * half;
            if (jt < IT) {
                const float4 fv = *(const float4*)&S.f[IT - 1][j0];
                fac[4 * gq] = fv.x; fac[4 * gq + 1] = fv.y; fac[4 * gq + 2] = fv.z; fac[4 * gq + 3] = fv.w;
            } else {
                const float4 sv = *(const float4*)&S.sc[j0];
                const float4 cv = *(const float4*)&S.cs2[j0];
                const float4 tv = *(const float4*)&S.st[j0];
                const float sa[4] = {sv.x, sv.y, sv.z, sv.w}, ca[4] = {cv.x, cv.y, cv.z, cv.w};
                const float ta[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float tj = ta[e];
                    // exponent clamped at 0: only the tj < ti entries are kept
                    const float k = sa[e] * __builtin_amdgcn_exp2f(fminf(cs_i - ca[e], 0.f));
                    fac[4 * gq + e] = tj < ti ? k : (tj == ti ? gm_i : 0.f);
                }
            }
        }
        if (jt == IT) {
            const float el = __builtin_amdgcn_exp2f(cs_i - cs_r0);
#pragma unroll
            for (int v = 0; v < 16; ++v) y[v] *= el;
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            s3_bf16x8_t bop, bopl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 hi, lo;
                s3_split(d[8 * kk + e], fac[8 * kk + e], hi, lo);
                bop[e] = hi;
                bopl[e] = lo;
            }
            // v^T[p][j] in the same permuted k order: j = 32 jt + 16 kk + 4 half + {0..3, 8..11}
            const int j0 = jt * 32 + 16 * kk + 4 * half;
            const s3_bf16x4_t lo = *(const s3_bf16x4_t*)&S.xT[r][j0];
            const s3_bf16x4_t hi = *(const s3_bf16x4_t*)&S.xT[r][j0 + 8];
            const s3_bf16x8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            y = s3_mfma(a, bop, y);
            y = s3_mfma(a, bopl, y);
        }
    }
}

// The chunk-entry state of one wave's dstate tile (columns 32 nt .. 32 nt + 31,
// accumulator layout: row 8 (v / 4) + 4 half + v % 4, column r) into buffer
// `buf` as hi + lo.
template <int QF, int HB, int NY>
__device__ __forceinline__ void ssd3_put_state(Ssd3Lds<QF, HB, NY>& S, const s3_f32x16_t& h, int buf, int nt, int r,
                                               int half) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = 8 * (v >> 2) + 4 * half + (v & 3);
        S.h[buf][row][nt * 32 + r] = __builtin_bit_cast(bf16_t, s3_h16(h[v]));
        S.hl[buf][row][nt * 32 + r] = __builtin_bit_cast(bf16_t, s3_l16(h[v]));
    }
}

// One wave's state update h <- h + sum_j (w_j v^T[p][j]) B[j][n] over the
// chunk (the caller has applied exp(cs_end)), n tile = nt; the B operand is
// gathered column-wise from the row-major B tile, the weighted v^T enters as
// hi + lo.
template <int QF, int HB, int NY>
__device__ __forceinline__ void ssd3_state_update(Ssd3Lds<QF, HB, NY>& S, s3_f32x16_t& h, int nt, int r, int half) {
    constexpr int KS = QF / 16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int j0 = ks * 16 + 8 * half;
        const s3_bf16x8_t a = *(const s3_bf16x8_t*)&S.xTw[r][j0];
        const s3_bf16x8_t al = *(const s3_bf16x8_t*)&S.xTwl[r][j0];
        s3_bf16x8_t bo;
#pragma unroll
        for (int e = 0; e < 8; ++e) bo[e] = __builtin_bit_cast(__bf16, S.B[j0 + e][nt * 32 + r]);
        h = s3_mfma(a, bo, h);
        h = s3_mfma(al, bo, h);
    }
}

}  // namespace mamba
