// Mamba-3 prefill prologue fused into the single-SSD scan, gfx950 MFMA path.
//
// Reference: Mamba3::forward_single_ssd (burn-mamba
// src/mamba3/single_ssd/single_ssd/mod.rs:86-290): steps 2-6 (trapezoidal
// coefficients helpers.rs:42-73 and scale_t = gamma_t + (1 - lambda_{t+1})
// dt_{t+1} :129-150; qk_norm_expand_bias helpers.rs:82-95; rotate_bc_forward
// Complex2D rotation/mod.rs:653-679; v = x mimo_x helpers.rs:152-168) feed
// step 7's single_ssd_serial_recalculated
// (single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-291), and step
// 9 adds D v.
//
// The scan is the one of ssd3_mfma.hip (one workgroup of 4 waves per (batch,
// head, 32-wide headdim half), chunks of QF = 128 fused positions f = M t + m,
// the state in MFMA accumulators), but its loaders read the raw in_proj row:
//   * coefficients: each fused position's thread forms dt, da, lambda of its
//     step (and dt, lambda of the next step for scale) from dd_dt, dd_A,
//     lambda_raw; da enters the chunk's cumulative sum once per step;
//   * angles: thread (a, q) takes angle a over an eighth of the chunk's steps:
//     increments dt range pi tanh(rot) on the fixed-point angle grid of
//     mamba3_internal.h, a local running sum, the eighths' exclusive prefix by
//     DPP inside the group of 8, the carried angle added; cos / sin go to an LDS
//     table [step][pair] (1, 0 past the rotated pairs), and the chunk's last
//     angle is carried to the next chunk;
//   * B rows (row-major LDS tile, the shared MFMA operand): RMS over the row's
//     16 lanes, norm weight and per-(head, rank) bias, the (k, k + N/2)
//     rotation with the partner column from lane ^ 8, rounded to bf16; at
//     MIMO rank 1 (SISO) the (2k, 2k + 1) rotation inside the lane, with the
//     angles tabulated per (step, pair) and their cos / sin formed by the row
//     threads (a per-step cos / sin table of 128 steps does not fit in LDS);
//   * C rows (each wave's MFMA fragments, in registers): the same, the RMS
//     completed with lane ^ 32 and both rotation partners in the same lane;
//   * v^T = (x mimo_x)^T and its w-scaled copy from the x columns.
// The epilogue adds D v to y.  The cache tail (last step's rotated B and x,
// the wrapped last angle) is written from the same registers.  The beta seed
// of the initial state runs before, in mamba3_prep.hip's seed kernel.
#include "mamba3_internal.h"
#include "ssd3_core.h"

namespace mamba {

struct M3FusedParams {
    int nb, L, H, G, A, npair, nch;
    const bf16_t* proj; int64_t proj_sb, proj_sl;  // elements
    int o_x, o_b, o_c, o_dt;                       // row offsets: x, B, C, dd_dt (dd_A +H, lambda +2H, rot +3H)
    const float* dt_bias; float a_floor, dt_lo, dt_hi, span;
    const float* bnw; const float* cnw; const float* bbias; const float* cbias; const float* mx; const float* Dh;
    const float* ang; float* ang_out; float* kst; float* vst;
    const float* h0; float* hT;
    bf16_t* y;  // [b, L, M, H, 64] contiguous
};

// y staged in LDS for whole-line stores, except at M = 1 and 2, whose angle
// or cos / sin tables leave no room for the staging tiles: y is then stored
// straight from the accumulators (8 bytes per lane and row)
template <int M>
constexpr int m3f_ny() { return M <= 2 ? 1 : 4; }

template <int M>
struct __align__(16) M3FusedLds {
    static constexpr int TS = 128 / M;                   // steps per chunk
    static constexpr int TCS = M == 1 ? 1 : TS;          // rows of the cos / sin tables
    Ssd3Lds<128, 1, m3f_ny<M>()> core;  // one chunk-entry state buffer: written at the next chunk's start
    bf16_t C[128][136];                  // C rows of the chunk (the y tiles' MFMA B operand)
    float cs[TCS][64], sn[TCS][64];      // M > 1: cos / sin per step and pair index k, at m3f_pos(k)
    int ang[M == 1 ? TS : 1][64];        // M = 1: the angle per step and pair index k (grid units)
    float4 bwb[M][4][16], cwb[M][4][16];  // (w, bias, w, bias) of columns 8 nv + 2 e2 (+1) of B / C
                                          // per rank, at [m][e2][nv]
    float mx[M][32];                      // mimo_x of this headdim half
    float dt[TS];                         // dt per step of the chunk (0 past the end)
};

__device__ __forceinline__ float m3f_bf(uint32_t u) { return __uint_as_float(u << 16); }
// Position of pair index k in a cos / sin table row: the four entries 8 j .. 8 j + 3
// at 4 j, the four 8 j + 4 .. 8 j + 7 at 32 + 4 j.  A thread whose columns hold the
// pairs 8 j .. 8 j + 7 reads them as two 16-byte vectors, and the 8 threads j = 0..7
// of a row read 32 consecutive dwords per instruction (no bank conflicts).
__device__ __forceinline__ int m3f_pos(int k) { return ((k & 4) << 3) + ((k >> 3) << 2) + (k & 3); }
// value of lane ^ 8 inside a 16-lane row (row_ror:8; every lane is written)
__device__ __forceinline__ float m3f_xor8(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
}
// value of lane - K inside a 16-lane row (row_shr:K), 0 where that leaves the row
template <int K>
__device__ __forceinline__ int m3f_shr(int x) {
    return __builtin_amdgcn_update_dpp(0, x, 0x110 + K, 0xf, 0xf, false);
}
// value of lane 8 (lane / 8) + 7: the last lane of each aligned group of 8 (ds_swizzle bit masks)
__device__ __forceinline__ int m3f_last8(int x) { return __builtin_amdgcn_ds_swizzle(x, 0x18 | (0x7 << 5)); }

// Two rows (ranks m0 and m0 + 1 of one step) x 8 columns (8 nv ..) of raw
// group-form B or C: the RMS over the row's 16 lanes, norm weight and bias,
// the (k, k + N/2) rotation with the partner columns from lane ^ 8 (k = n mod
// N/2; cs / sn point at the step's table entries for this thread's first four
// pairs, the next four 32 entries on: the m3f_pos layout).  The arithmetic is
// mamba3_internal.h's, as in the segment prep: the same bits.
// Writes the bf16 rows to the LDS tile and leaves the f32 rows in y0 / y1.
__device__ __forceinline__ void m3f_rows(uint4 r0, uint4 r1, const float (&w)[8], const float (&b0)[8],
                                         const float (&b1)[8], const float* cs, const float* sn, float sgn,
                                         bf16_t* dst0, bf16_t* dst1, float (&y0)[8], float (&y1)[8]) {
    const uint32_t a0[4] = {r0.x, r0.y, r0.z, r0.w}, a1[4] = {r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        y0[2 * e] = s3_lo(a0[e]); y0[2 * e + 1] = s3_hi(a0[e]);
        y1[2 * e] = s3_lo(a1[e]); y1[2 * e + 1] = s3_hi(a1[e]);
    }
    const float ss0 = m3_group_sum<16>(m3_sumsq8(y0));
    const float ss1 = m3_group_sum<16>(m3_sumsq8(y1));
    const float rms0 = m3_rms_inv(ss0, 128), rms1 = m3_rms_inv(ss1, 128);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        y0[e] = m3_norm(y0[e], rms0, w[e], b0[e]);
        y1[e] = m3_norm(y1[e], rms1, w[e], b1[e]);
    }
    float o0[8], o1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        o0[e] = m3f_xor8(y0[e]);
        o1[e] = m3f_xor8(y1[e]);
    }
    const float4 c0 = *(const float4*)cs, c1 = *(const float4*)(cs + 32);
    const float4 s0 = *(const float4*)sn, s1 = *(const float4*)(sn + 32);
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        y0[e] = m3_rot(cv[e], y0[e], sgn * sv[e], o0[e]);
        y1[e] = m3_rot(cv[e], y1[e], sgn * sv[e], o1[e]);
    }
    *(uint4*)dst0 = make_uint4(pack_bf16x2(y0[0], y0[1]), pack_bf16x2(y0[2], y0[3]), pack_bf16x2(y0[4], y0[5]),
                               pack_bf16x2(y0[6], y0[7]));
    *(uint4*)dst1 = make_uint4(pack_bf16x2(y1[0], y1[1]), pack_bf16x2(y1[2], y1[3]), pack_bf16x2(y1[4], y1[5]),
                               pack_bf16x2(y1[6], y1[7]));
}

// Two consecutive steps' rows at M = 1 x 8 columns: the RMS, weight and bias
// as m3f_rows, then the (2k, 2k + 1) rotation inside the lane with the cos /
// sin of the thread's pairs 4 nv .. 4 nv + 3 of each row's step (c0 / s0,
// c1 / s1), as the segment prep rotates SISO rows.
__device__ __forceinline__ void m3f_rows1(uint4 r0, uint4 r1, const float (&w)[8], const float (&bias)[8],
                                          const float (&c0)[4], const float (&s0)[4], const float (&c1)[4],
                                          const float (&s1)[4], bf16_t* dst0, bf16_t* dst1, float (&y0)[8],
                                          float (&y1)[8]) {
    const uint32_t a0[4] = {r0.x, r0.y, r0.z, r0.w}, a1[4] = {r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        y0[2 * e] = s3_lo(a0[e]); y0[2 * e + 1] = s3_hi(a0[e]);
        y1[2 * e] = s3_lo(a1[e]); y1[2 * e + 1] = s3_hi(a1[e]);
    }
    const float ss0 = m3_group_sum<16>(m3_sumsq8(y0));
    const float ss1 = m3_group_sum<16>(m3_sumsq8(y1));
    const float rms0 = m3_rms_inv(ss0, 128), rms1 = m3_rms_inv(ss1, 128);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        y0[e] = m3_norm(y0[e], rms0, w[e], bias[e]);
        y1[e] = m3_norm(y1[e], rms1, w[e], bias[e]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float u0 = y0[2 * j], u1 = y0[2 * j + 1];
        y0[2 * j] = m3_rot(c0[j], u0, -s0[j], u1);
        y0[2 * j + 1] = m3_rot(c0[j], u1, s0[j], u0);
        const float v0 = y1[2 * j], v1 = y1[2 * j + 1];
        y1[2 * j] = m3_rot(c1[j], v0, -s1[j], v1);
        y1[2 * j + 1] = m3_rot(c1[j], v1, s1[j], v0);
    }
    *(uint4*)dst0 = make_uint4(pack_bf16x2(y0[0], y0[1]), pack_bf16x2(y0[2], y0[3]), pack_bf16x2(y0[4], y0[5]),
                               pack_bf16x2(y0[6], y0[7]));
    *(uint4*)dst1 = make_uint4(pack_bf16x2(y1[0], y1[1]), pack_bf16x2(y1[2], y1[3]), pack_bf16x2(y1[4], y1[5]),
                               pack_bf16x2(y1[6], y1[7]));
}

// M bf16 values to LDS as one store (2 M bytes, aligned to its size)
template <int M>
__device__ __forceinline__ void m3f_st(bf16_t* dst, const float* v) {
    if constexpr (M == 1) {
        *dst = __builtin_bit_cast(bf16_t, s3_h16(v[0]));  // the hardware conversion, as for M > 1
    } else if constexpr (M == 2) {
        *(uint32_t*)dst = pack_bf16x2(v[0], v[1]);
    } else if constexpr (M == 4) {
        *(uint2*)dst = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
        *(uint4*)dst = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                  pack_bf16x2(v[6], v[7]));
    }
}

// 8 waves, two per SIMD: all take part in the chunk's prologue (coefficients,
// angles, B and C rows, v^T); then waves 0-3 compute the y tiles (tile =
// wave) while waves 4-7 update the state (dstate columns 32 (wave - 4) ..).
template <int M>
__global__ __launch_bounds__(512, 1) void mamba3_ssd_fused(M3FusedParams p) {
    constexpr int QF = 128, N = 128;
    constexpr int TS = QF / M;                    // steps per chunk
    constexpr int lgM = M == 1 ? 0 : M == 2 ? 1 : (M == 4 ? 2 : 3);
    static_assert(M == 1 || M == 2 || M == 4 || M == 8, "MIMO rank 1, 2, 4 or 8");
    constexpr int JA = TS / 8;                    // steps per angle thread (8 threads per angle)
    constexpr int XI = TS * 8, XPT = (XI + 511) / 512;  // x items: (step, 4-wide headdim piece)
    constexpr int RP = 2;                         // B row pairs and C row pairs per thread
    constexpr bool STAGE_Y = m3f_ny<M>() == 4;
    __shared__ M3FusedLds<M> SF;
    Ssd3Lds<QF, 1, m3f_ny<M>()>& S = SF.core;

    const int tid_ = threadIdx.x, r_ = tid_ & 31, half_ = (tid_ >> 5) & 1;
    const int wv = wave_id(), w4 = wv & 3;
    // XCD-aware mapping: the two headdim halves of a head and neighbouring heads on one XCD
    const int nwg = p.nb * p.H * 2;
    int w = blockIdx.x;
    if ((nwg & 7) == 0) w = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    const int ph = w & 1, h = (w >> 1) % p.H, b = (w >> 1) / p.H;
    const int g = h / (p.H / p.G);
    const int p0 = ph * 32;
    const int64_t bh = (int64_t)b * p.H + h;

    // per-head constants
    for (int i = tid_; i < M * 64; i += 512) {
        const int m = i >> 6, nv = (i >> 2) & 15, e2 = i & 3, n = nv * 8 + 2 * e2;
        const float* bb = p.bbias + ((int64_t)h * M + m) * N;
        const float* cb = p.cbias + ((int64_t)h * M + m) * N;
        SF.bwb[m][e2][nv] = make_float4(p.bnw[n], bb[n], p.bnw[n + 1], bb[n + 1]);
        SF.cwb[m][e2][nv] = make_float4(p.cnw[n], cb[n], p.cnw[n + 1], cb[n + 1]);
    }
    if (tid_ < M * 32) {
        const int m = tid_ >> 5, pp = tid_ & 31;
        SF.mx[m][pp] = p.mx ? p.mx[((int64_t)h * M + m) * 64 + p0 + pp] : 1.f;
    }
    // state tile of waves 4-7: headdim rows p0..p0+31, dstate columns 32 w4..
    s3_f32x16_t hacc;
    const int64_t hbase = bh * 64 * N;
    if (wv >= 4) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int pp = p0 + 8 * (v >> 2) + 4 * half_ + (v & 3);
            hacc[v] = p.h0[hbase + pp * N + w4 * 32 + r_];
        }
        ssd3_put_state(S, hacc, 0, w4, r_, half_);
    }

    const float dtb = p.dt_bias[h];
    const float Dv = p.Dh ? p.Dh[h] : 0.f;
    const bf16_t* projb = p.proj + (int64_t)b * p.proj_sb;
    const uint32_t rs = (uint32_t)p.proj_sl * 2;  // bytes per proj row (the host bounds (TS + 1) rows below 2^31)
    bf16_t* yhead = p.y + (int64_t)b * p.L * M * p.H * 64 + (int64_t)h * 64 + p0;
    const uint32_t y_rs = (uint32_t)p.H * 64 * 2;

    // ---- thread roles and their byte offsets within a chunk's proj rows
    // coefficients: fused position f = tid (< QF) of step f >> lgM
    const uint32_t co_dt = (uint32_t)((tid_ & (QF - 1)) >> lgM) * rs + (uint32_t)(p.o_dt + h) * 2;
    const uint32_t co_da = co_dt + (uint32_t)p.H * 2, co_lam = co_dt + (uint32_t)p.H * 4;
    // angles: a = tid / 8 over steps q JA .. q JA + JA - 1, q = tid % 8
    const uint32_t ao = (uint32_t)((tid_ & 7) * JA) * rs + (uint32_t)(p.o_dt + 3 * p.H + min(tid_ >> 3, p.A - 1)) * 2;
    // B and C rows: pairs fp = tid / 16 + 32 k (rows 2 fp, 2 fp + 1: ranks bm0, bm0 + 1 of one
    // step; at M = 1 steps 2 fp and 2 fp + 1), columns 8 nv .. 8 nv + 7
    const uint32_t bro = (uint32_t)((2 * (tid_ >> 4)) >> lgM) * rs +
                         (uint32_t)((((2 * (tid_ >> 4)) & (M - 1)) * p.G + g) * N + (tid_ & 15) * 8) * 2;
    const uint32_t bo = bro + (uint32_t)p.o_b * 2, cofs = bro + (uint32_t)p.o_c * 2;
    // the pair's second row: rank bm0 + 1 of the step, or at M = 1 the next step's row
    const uint32_t r2 = M == 1 ? rs : (uint32_t)p.G * N * 2;

    // ---- register prefetch of one chunk's raw proj data
    uint2 xq[XPT];
    uint4 bq[RP][2], cq[RP][2];
    uint32_t kq[5] = {0u, 0u, 0u, 0u, 0u};
    uint32_t rq[JA];
    // rows of chunk c and the step after it (scale's shift); zero past the end
    auto chunk_rsrc = [&](int c) {
        const int steps = max(0, min(TS + 1, p.L - c * TS));  // none past the last chunk
        return buf_rsrc(projb + (int64_t)c * TS * p.proj_sl, (uint32_t)steps * rs);
    };
    auto fetch_rows = [&](int c) {
        const __amdgpu_buffer_rsrc_t rp = chunk_rsrc(c);
#pragma unroll
        for (int k = 0; k < RP; ++k) {
            const uint32_t o = (uint32_t)((64 * k) >> lgM) * rs;
            bq[k][0] = buf_ld16(rp, bo + o);
            bq[k][1] = buf_ld16(rp, bo + o + r2);
            cq[k][0] = buf_ld16(rp, cofs + o);
            cq[k][1] = buf_ld16(rp, cofs + o + r2);
        }
    };
    auto fetch = [&](int c) {
        const __amdgpu_buffer_rsrc_t rp = chunk_rsrc(c);
        // every load is issued by every thread on every chunk (the threads past
        // the x items and positions load duplicates; past the last chunk the
        // resource is empty): the compiler's waits then count the same loads on
        // every path
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = (tid_ + 512 * k) % XI;
            xq[k] = buf_ld8(rp, (uint32_t)(item >> 3) * rs + (uint32_t)(p.o_x + h * 64 + p0 + (item & 7) * 4) * 2);
        }
        kq[0] = buf_ld2(rp, co_dt);
        kq[1] = buf_ld2(rp, co_da);
        kq[2] = buf_ld2(rp, co_lam);
        kq[3] = buf_ld2(rp, co_dt + rs);
        kq[4] = buf_ld2(rp, co_lam + rs);
#pragma unroll
        for (int j = 0; j < JA; ++j) rq[j] = buf_ld2(rp, ao + (uint32_t)j * rs);
    };
    // y tile of chunk c (waves 0-3) from its LDS staging: 32 rows x 64 bytes, 4 lanes per row
    auto store_y = [&](int c, int lane) {
        const int t0 = c * TS;
        const int rows = min(QF, (p.L - t0) * M);
        const __amdgpu_buffer_rsrc_t ry = buf_rsrc(yhead + (int64_t)t0 * M * p.H * 64, (uint32_t)rows * y_rs);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int row = q * 16 + (lane >> 2), ch = lane & 3;
            const uint4 val = *(const uint4*)&S.y[wv][row][ch * 8];
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(decltype(__builtin_amdgcn_raw_buffer_load_b128(ry, 0, 0, 0)), val), ry,
                (uint32_t)(wv * 32 + row) * y_rs + ch * 16, 0, 0);
        }
    };
    // the same issue order as inside the loop (small loads, then rows): the
    // waits at the loop head then count the same way on entry and on the back-edge
    // the cumulative angle of this thread's angle (grid units, mamba3_internal.h): loaded
    // before the prefetch
    int theta = (tid_ >> 3) < p.A ? m3_ang_fix(p.ang[bh * p.A + (tid_ >> 3)]) : 0;
    fetch(0);
    __builtin_amdgcn_sched_barrier(0);
    fetch_rows(0);
    __builtin_amdgcn_sched_barrier(0);

    // ---- A, on waves 4-5 (fused position tid - 256): coefficients of the
    // position from the raw columns of chunk cc (kq), SF.dt, and the block scan
    // of da (the two waves' totals and the tile anchors into LDS); the values
    // the tables need stay in this thread's registers until phase B
    float loc_a = 0.f, scq_a = 0.f, gmq_a = 0.f;
    auto phase_a = [&](int cc, int tid) __attribute__((always_inline)) {
        const int cf_tl = (tid & (QF - 1)) >> lgM;
        const bool cf_first = (tid & (M - 1)) == 0;
        float daq = 0.f, scq = 0.f, gmq = 0.f;
        const int t = cc * TS + cf_tl;
        float dt = 0.f;
        if (t < p.L) {
            float da, lam;
            m3_coef(m3f_bf(kq[0]), m3f_bf(kq[1]), m3f_bf(kq[2]), dtb, p.a_floor, p.dt_lo, p.dt_hi, dt, da, lam);
            float dt1 = 0.f, lam1 = 0.f;  // the next step's (scale's shift); 0 past the end
            if (t + 1 < p.L) {
                dt1 = fminf(fmaxf(m3p_softplus(m3f_bf(kq[3]) + dtb), p.dt_lo), p.dt_hi);
                lam1 = m3_sigmoid(m3f_bf(kq[4]));
            }
            gmq = lam * dt;
            scq = __builtin_fmaf(1.f - lam1, dt1, gmq);
            daq = cf_first ? da : 0.f;  // da enters the cumulative sum once per step
        }
        if (cf_first) SF.dt[cf_tl] = dt;
        const float loc = wave_incl_scan(daq * kLog2eS3);
        if ((tid & 63) == 63) S.red[(tid >> 6) - 4] = loc;
        if ((tid & 31) == 0) S.anc[(tid - 256) >> 5] = loc;
        loc_a = loc;
        scq_a = scq;
        gmq_a = gmq;
    };
    if (wv == 4 || wv == 5) phase_a(0, tid_);
    __syncthreads();

    for (int c = 0; c < p.nch; ++c) {
        const int t0 = c * TS;
        // thread coordinates redefined per chunk: LDS addresses derived from them are
        // formed inside the loop instead of being hoisted (and spilled) as invariants
        int tid = tid_;
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, r = lane & 31, half = lane >> 5;
        const int ang_a = tid >> 3, ang_q = tid & 7;
        const int b_fp = tid >> 4, b_nv = tid & 15;
        const int bm0 = (2 * b_fp) & (M - 1);
        const int kq4 = (b_nv & 7) * 4;  // m3f_pos of the thread's first pair index 8 (nv & 7)
        const float sgn = b_nv < 8 ? -1.f : 1.f;
        // ---- the state entering this chunk into its one LDS buffer (waves 4-7;
        // the y tiles of the previous chunk have read it before the last barrier,
        // this chunk's read it after the next one)
        if (c > 0 && wv >= 4) ssd3_put_state(S, hacc, 0, w4, r, half);
        // ---- A ran for this chunk on waves 4-5 during the previous chunk's
        // MFMA phase (phase_a below; before the loop for chunk 0)
        // ---- B: per-position tables (waves 4-5, whose registers hold phase
        // A's values); angles and their cos / sin
        const float cs_end = S.red[0] + S.red[1];
        if (wv == 4 || wv == 5) {
            const int j = tid - 256;
            const float csj = loc_a + (wv == 5 ? S.red[0] : 0.f);
            S.cs2[j] = csj;
            S.st[j] = (float)(j >> lgM);
            S.sc[j] = scq_a;
            S.gm[j] = gmq_a;
            S.w[j] = scq_a * __builtin_amdgcn_exp2f(cs_end - csj);
#pragma unroll
            for (int it = 1; it < 4; ++it) {
                if (j < it * 32) {
                    const float anchor = S.anc[it] + (it >= 2 ? S.red[0] : 0.f);
                    S.f[it - 1][j] = scq_a * __builtin_amdgcn_exp2f(anchor - csj);
                }
            }
        }
        {
            // increments on the fixed-point angle grid: integer sums, so every
            // position's angle is the one the segment prep forms
            // (every term canonical, |.| <= pi on the grid: the partial sums
            // below stay far from int32 overflow)
            int cum[JA];
            int run = 0;
#pragma unroll
            for (int j = 0; j < JA; ++j) {
                run += m3_ang_fix(m3_angle_inc(SF.dt[ang_q * JA + j], m3f_bf(rq[j]), p.span));
                cum[j] = run;
            }
            run = m3_ang_reduce(run);
            // inclusive scan of the 8 parts' (reduced) totals inside each aligned group of 8 lanes
            int incl = run;
            {
                const int t1 = m3f_shr<1>(incl);
                incl += ang_q >= 1 ? t1 : 0;
                const int t2 = m3f_shr<2>(incl);
                incl += ang_q >= 2 ? t2 : 0;
                const int t4 = m3f_shr<4>(incl);
                incl += ang_q >= 4 ? t4 : 0;
            }
            const int base = theta + (incl - run);
            const int total = m3f_last8(incl);
            const bool rot_on = ang_a < p.npair;
            if constexpr (M == 1) {
                // the angles themselves; the row threads form their cos / sin
                if (ang_a < 64)
#pragma unroll
                    for (int j = 0; j < JA; ++j) SF.ang[ang_q * JA + j][ang_a] = m3_ang_reduce(base + cum[j]);
            } else {
#pragma unroll
                for (int j = 0; j < JA; ++j) {
                    float c = 1.f, sn = 0.f;
                    if (rot_on) m3_cossin(m3_ang_rad(m3_ang_reduce(base + cum[j])), c, sn);
                    SF.cs[ang_q * JA + j][m3f_pos(ang_a)] = c;
                    SF.sn[ang_q * JA + j][m3f_pos(ang_a)] = sn;
                }
            }
            theta = m3_ang_reduce(theta + total);  // the chunk's last angle
        }
        __syncthreads();
        if constexpr (STAGE_Y)
            if (c > 0 && wv < 4) store_y(c - 1, lane);
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = tid + 512 * k;
            if (XI % 512 == 0 || item < XI) {
                const int tl = item >> 3, pv = item & 7;
                const float xv[4] = {s3_lo(xq[k].x), s3_hi(xq[k].x), s3_lo(xq[k].y), s3_hi(xq[k].y)};
                if (t0 + tl == p.L - 1)  // the cache tail: the last step's x
                    *(float4*)(p.vst + bh * 64 + p0 + pv * 4) = make_float4(xv[0], xv[1], xv[2], xv[3]);
                float vt[4][M], vw[4][M], vwl[4][M];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float wf = S.w[tl * M + m];
                    const float4 mv = *(const float4*)&SF.mx[m][pv * 4];
                    const float mxa[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float vb = (float)(__bf16)(xv[e] * mxa[e]);  // v as the SSD seam holds it (bf16)
                        vt[e][m] = vb;
                        // w v as hi + lo, split as the seam splits it (hi exact in bf16, lo
                        // rounded by the store)
                        vw[e][m] = (float)(__bf16)(vb * wf);
                        vwl[e][m] = s3_res(vb, wf, vw[e][m]);
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    m3f_st<M>(&S.xT[pv * 4 + e][tl * M], vt[e]);
                    m3f_st<M>(&S.xTw[pv * 4 + e][tl * M], vw[e]);
                    m3f_st<M>(&S.xTwl[pv * 4 + e][tl * M], vwl[e]);
                }
            }
        }
        // the next chunk's coefficient, angle and x columns (their registers are free now)
        __builtin_amdgcn_sched_barrier(0);
        fetch(c + 1);
        __builtin_amdgcn_sched_barrier(0);
        // ---- C: B and C rows to LDS; v^T and w-scaled v^T
        if constexpr (M == 1) {
            float bw[8], bb[8], cw[8], cb[8];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float4 u = SF.bwb[0][e >> 1][b_nv], v = SF.cwb[0][e >> 1][b_nv];
                bw[e] = u.x; bb[e] = u.y; bw[e + 1] = u.z; bb[e + 1] = u.w;
                cw[e] = v.x; cb[e] = v.y; cw[e + 1] = v.z; cb[e + 1] = v.w;
            }
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                const int f0 = 2 * (b_fp + 32 * k);  // steps f0 and f0 + 1 of the chunk
                // cos / sin of the thread's pairs 4 nv .. 4 nv + 3 at both steps ((1, 0) past
                // the rotated pairs)
                float c0[4], s0[4], c1[4], s1[4];
                const int4 q0 = *(const int4*)&SF.ang[f0][4 * b_nv], q1 = *(const int4*)&SF.ang[f0 + 1][4 * b_nv];
                const int qa0[4] = {q0.x, q0.y, q0.z, q0.w}, qa1[4] = {q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    c0[j] = 1.f; s0[j] = 0.f; c1[j] = 1.f; s1[j] = 0.f;
                    if (4 * b_nv + j < p.npair) {
                        m3_cossin(m3_ang_rad(qa0[j]), c0[j], s0[j]);
                        m3_cossin(m3_ang_rad(qa1[j]), c1[j], s1[j]);
                    }
                }
                float y0[8], y1[8];
                m3f_rows1(bq[k][0], bq[k][1], bw, bb, c0, s0, c1, s1, &S.B[f0][b_nv * 8], &S.B[f0 + 1][b_nv * 8],
                          y0, y1);
                // the cache tail: the last step's rotated B (f32)
                if (ph == 0 && t0 + f0 + 1 >= p.L - 1 && t0 + f0 <= p.L - 1) {
                    const float* yl = t0 + f0 == p.L - 1 ? y0 : y1;
                    float* k0 = p.kst + ((int64_t)b * p.H + h) * N + b_nv * 8;
                    *(float4*)k0 = make_float4(yl[0], yl[1], yl[2], yl[3]);
                    *(float4*)(k0 + 4) = make_float4(yl[4], yl[5], yl[6], yl[7]);
                }
                m3f_rows1(cq[k][0], cq[k][1], cw, cb, c0, s0, c1, s1, &SF.C[f0][b_nv * 8], &SF.C[f0 + 1][b_nv * 8],
                          y0, y1);
            }
        } else {
            float bw[8], bb0[8], bb1[8], cw[8], cb0[8], cb1[8];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float4 u0 = SF.bwb[bm0][e >> 1][b_nv], u1 = SF.bwb[bm0 + 1][e >> 1][b_nv];
                const float4 v0 = SF.cwb[bm0][e >> 1][b_nv], v1 = SF.cwb[bm0 + 1][e >> 1][b_nv];
                bw[e] = u0.x; bb0[e] = u0.y; bw[e + 1] = u0.z; bb0[e + 1] = u0.w;
                bb1[e] = u1.y; bb1[e + 1] = u1.w;
                cw[e] = v0.x; cb0[e] = v0.y; cw[e + 1] = v0.z; cb0[e + 1] = v0.w;
                cb1[e] = v1.y; cb1[e + 1] = v1.w;
            }
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                const int f0 = 2 * (b_fp + 32 * k), tl = f0 >> lgM;
                float y0[8], y1[8];
                m3f_rows(bq[k][0], bq[k][1], bw, bb0, bb1, &SF.cs[tl][kq4], &SF.sn[tl][kq4], sgn,
                         &S.B[f0][b_nv * 8], &S.B[f0 + 1][b_nv * 8], y0, y1);
                // the cache tail: the last step's rotated B (f32)
                if (ph == 0 && t0 + tl == p.L - 1) {
                    float* k0 = p.kst + (((int64_t)b * M + bm0) * p.H + h) * N + b_nv * 8;
                    float* k1 = p.kst + (((int64_t)b * M + bm0 + 1) * p.H + h) * N + b_nv * 8;
                    *(float4*)k0 = make_float4(y0[0], y0[1], y0[2], y0[3]);
                    *(float4*)(k0 + 4) = make_float4(y0[4], y0[5], y0[6], y0[7]);
                    *(float4*)k1 = make_float4(y1[0], y1[1], y1[2], y1[3]);
                    *(float4*)(k1 + 4) = make_float4(y1[4], y1[5], y1[6], y1[7]);
                }
                m3f_rows(cq[k][0], cq[k][1], cw, cb0, cb1, &SF.cs[tl][kq4], &SF.sn[tl][kq4], sgn,
                         &SF.C[f0][b_nv * 8], &SF.C[f0 + 1][b_nv * 8], y0, y1);
            }
        }
        // ---- the next chunk's rows land during this chunk's MFMA work
        __builtin_amdgcn_sched_barrier(0);
        fetch_rows(c + 1);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        if (wv >= 4) {
            // ---- D (waves 4-7): h <- exp(cs_end) h + sum_j (w_j v^T[p][j]) B[j][n], n tile = w4
            const float dec = __builtin_amdgcn_exp2f(cs_end);
#pragma unroll
            for (int v = 0; v < 16; ++v) hacc[v] *= dec;
            ssd3_state_update(S, hacc, w4, r, half);
            // ---- A of the next chunk (its raw columns were fetched in phase C;
            // SF.dt, S.red and S.anc were last read in this chunk's phase B)
            if ((wv == 4 || wv == 5) && c + 1 < p.nch) phase_a(c + 1, tid);
        } else {
            // ---- D (waves 0-3): y for output tile = wave, plus D v
            s3_bf16x8_t cfr[8];
#pragma unroll
            for (int kn = 0; kn < 8; ++kn) cfr[kn] = *(const s3_bf16x8_t*)&SF.C[wv * 32 + r][kn * 16 + 8 * half];
            s3_f32x16_t yacc;
            switch (wv) {
                case 0: ssd3_y_tile<QF, 0, true>(S, cfr, 0, r, half, yacc); break;
                case 1: ssd3_y_tile<QF, 1, true>(S, cfr, 0, r, half, yacc); break;
                case 2: ssd3_y_tile<QF, 2, true>(S, cfr, 0, r, half, yacc); break;
                default: ssd3_y_tile<QF, 3, true>(S, cfr, 0, r, half, yacc); break;
            }
            if (p.Dh) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int pp = 8 * (v >> 2) + 4 * half + (v & 3);
                    yacc[v] += Dv * bf16_to_f32(S.xT[pp][wv * 32 + r]);
                }
            }
            // lane holds y[i][p = 8(v/4) + 4 half + v%4]
            if constexpr (STAGE_Y) {
                // stage the 32 (position) x 32 (p) tile
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    const s3_bf16x4_t q = {(__bf16)yacc[4 * gq], (__bf16)yacc[4 * gq + 1], (__bf16)yacc[4 * gq + 2],
                                           (__bf16)yacc[4 * gq + 3]};
                    *(s3_bf16x4_t*)&S.y[wv][r][8 * gq + 4 * half] = q;
                }
                // stored from the staging tile during the next chunk (store_y), after that
                // chunk's waits on its prefetched loads, which then never wait on these stores
            } else {
                const int rows = min(QF, (p.L - t0) * M);
                const __amdgpu_buffer_rsrc_t ry = buf_rsrc(yhead + (int64_t)t0 * M * p.H * 64, (uint32_t)rows * y_rs);
#pragma unroll
                for (int gq = 0; gq < 4; ++gq)
                    buf_st8(ry, (uint32_t)(wv * 32 + r) * y_rs + (8 * gq + 4 * half) * 2,
                            make_uint2(pack_bf16x2(yacc[4 * gq], yacc[4 * gq + 1]),
                                       pack_bf16x2(yacc[4 * gq + 2], yacc[4 * gq + 3])));
            }
        }
        __syncthreads();  // LDS reads of this chunk done before the next commit
    }
    if constexpr (STAGE_Y)
        if (wv < 4) store_y(p.nch - 1, tid_ & 63);
    if (wv >= 4) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int pp = p0 + 8 * (v >> 2) + 4 * half_ + (v & 3);
            p.hT[hbase + pp * N + w4 * 32 + r_] = hacc[v];
        }
    }
    if (ph == 0 && (tid_ & 7) == 0 && (tid_ >> 3) < p.A) p.ang_out[bh * p.A + (tid_ >> 3)] = m3_ang_rad(theta);
}

// Validates the arguments (-1 with the error set when invalid), fills the
// prologue's and the scan's parameter blocks, and says whether the fused
// kernel covers this shape and layout.
static int m3_fused_params(const mamba3_fused_args* a, M3PrepParams* pp, M3FusedParams* fp, bool* ok) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    const int st = m3_prep_params(&a->prep, pp, false);
    if (st != MAMBA_OK) return st;
    MAMBA_CHECK_ARG(a->y && a->final_state, "y and final_state are required");
    const M3PrepParams& p = *pp;
    const int M = p.M;
    const int TS = M > 0 ? 128 / M : 0;
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    *ok = p.proj_bf16 && p.P == 64 && p.N == 128 && (M == 1 || M == 2 || M == 4 || M == 8) && al16(p.proj) &&
          al16(a->y) && al16(p.kst) && al16(p.vst) && p.proj_sl % 8 == 0 && (p.nb == 1 || p.proj_sb % 8 == 0) && p.A <= 64 &&
          (int64_t)(TS + 1) * p.proj_sl * 2 < (1ll << 31) && (int64_t)p.L * M < (1ll << 30) &&
          (int64_t)p.nb * p.H * 2 < (1ll << 31);
    M3FusedParams& f = *fp;
    f.nb = p.nb; f.L = p.L; f.H = p.H; f.G = p.G; f.A = p.A; f.npair = p.R / 2;
    f.nch = TS > 0 ? (p.L + TS - 1) / TS : 0;
    f.proj = static_cast<const bf16_t*>(p.proj); f.proj_sb = p.proj_sb; f.proj_sl = p.proj_sl;
    f.o_x = p.H * p.P; f.o_b = 2 * p.H * p.P; f.o_c = f.o_b + M * p.G * p.N; f.o_dt = f.o_c + M * p.G * p.N;
    f.dt_bias = p.dt_bias; f.a_floor = p.a_floor; f.dt_lo = p.dt_lo; f.dt_hi = p.dt_hi; f.span = p.span;
    f.bnw = p.bnw; f.cnw = p.cnw; f.bbias = p.bbias; f.cbias = p.cbias; f.mx = p.mx; f.Dh = a->D;
    f.ang = p.ang; f.ang_out = p.ang_out; f.kst = p.kst; f.vst = p.vst;
    f.h0 = p.h0; f.hT = a->final_state;
    f.y = static_cast<bf16_t*>(a->y);
    return MAMBA_OK;
}

static int m3_fused_run(const mamba3_fused_args* a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
    M3PrepParams pp;
    M3FusedParams fp;
    bool ok = false;
    const int st = m3_fused_params(a, &pp, &fp, &ok);
    if (st != MAMBA_OK) return st;
    MAMBA_CHECK_ARG(ok, "shape or layout outside the fused kernel (mamba3_ssd_fused_supported() == 0)");
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
    m3_launch_seed(pp, s);
    MAMBA_CHECK_LAUNCH();
    const dim3 grid(fp.nb * fp.H * 2), block(512);
    switch (pp.M) {
        case 1: hipLaunchKernelGGL(mamba3_ssd_fused<1>, grid, block, 0, s, fp); break;
        case 2: hipLaunchKernelGGL(mamba3_ssd_fused<2>, grid, block, 0, s, fp); break;
        case 4: hipLaunchKernelGGL(mamba3_ssd_fused<4>, grid, block, 0, s, fp); break;
        default: hipLaunchKernelGGL(mamba3_ssd_fused<8>, grid, block, 0, s, fp); break;
    }
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" int mamba3_ssd_fused_supported(const mamba3_fused_args* a) {
    M3PrepParams pp;
    M3FusedParams fp;
    bool ok = false;
    if (m3_fused_params(a, &pp, &fp, &ok) != MAMBA_OK) return -1;
    return ok ? 1 : 0;
}

extern "C" int mamba3_ssd_fused_fwd(const mamba3_fused_args* a, mamba_stream_t stream) {
    return m3_fused_run(a, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba3_ssd_fused_fwd_timed(const mamba3_fused_args* a, mamba_stream_t stream, void* event_start,
                                          void* event_stop) {
    return m3_fused_run(a, (hipStream_t)stream, (hipEvent_t)event_start, (hipEvent_t)event_stop);
}
