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
//   * angles: thread (a, q) takes angle a over a quarter of the chunk's steps:
//     increments dt range pi tanh(rot), a local running sum, the quarters'
//     exclusive prefix by DPP inside the quad, the carried angle added and
//     wrapped; cos / sin go to an LDS table [step][pair] (1, 0 past the rotated
//     pairs), and the chunk's last angle is carried to the next chunk;
//   * B rows (row-major LDS tile, the shared MFMA operand): RMS over the row's
//     16 lanes, norm weight and per-(head, rank) bias, the (k, k + N/2)
//     rotation with the partner column from lane ^ 8, rounded to bf16;
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

template <int M>
struct __align__(16) M3FusedLds {
    Ssd3Lds<128> core;
    float cs[128 / M][64], sn[128 / M][64];  // cos / sin per step of the chunk and pair index
    float2 bwb[M][128], cwb[M][128];         // (norm weight, bias) of B and C per rank and column
    float mx[M][32];                         // mimo_x of this headdim half
    float dt[128 / M];                       // dt per step of the chunk (0 past the end)
};

__device__ __forceinline__ float m3f_bf(uint32_t u) { return __uint_as_float(u << 16); }

// M bf16 values to LDS as one store (2 M bytes, aligned to its size)
template <int M>
__device__ __forceinline__ void m3f_st(bf16_t* dst, const float* v) {
    if constexpr (M == 2) {
        *(uint32_t*)dst = pack_bf16x2(v[0], v[1]);
    } else if constexpr (M == 4) {
        *(uint2*)dst = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
        *(uint4*)dst = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                  pack_bf16x2(v[6], v[7]));
    }
}

template <int M>
__global__ __launch_bounds__(256, 1) void mamba3_ssd_fused(M3FusedParams p) {
    constexpr int QF = 128, N = 128, NK = N / 16, KS = QF / 16;
    constexpr int TS = QF / M;                    // steps per chunk
    constexpr int lgM = M == 2 ? 1 : (M == 4 ? 2 : 3);
    static_assert(M == 2 || M == 4 || M == 8, "MIMO rank 2, 4 or 8");
    constexpr int JA = TS / 4;                    // steps per angle thread
    constexpr int XI = TS * 8, XPT = (XI + 255) / 256;  // x items: (step, 4-wide headdim piece)
    constexpr int BPT = 4;                        // B items: (row pair, 8-wide column piece)
    __shared__ M3FusedLds<M> SF;
    Ssd3Lds<QF>& S = SF.core;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 31, half = lane >> 5;
    // XCD-aware mapping: the two headdim halves of a head and neighbouring heads on one XCD
    const int nwg = p.nb * p.H * 2;
    int w = blockIdx.x;
    if ((nwg & 7) == 0) w = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    const int ph = w & 1, h = (w >> 1) % p.H, b = (w >> 1) / p.H;
    const int g = h / (p.H / p.G);
    const int p0 = ph * 32;
    const int64_t bh = (int64_t)b * p.H + h;

    // per-head constants
    for (int i = tid; i < M * N; i += 256) {
        const int m = i / N, n = i % N;
        const int64_t o = ((int64_t)h * M + m) * N + n;
        SF.bwb[m][n] = make_float2(p.bnw[n], p.bbias[o]);
        SF.cwb[m][n] = make_float2(p.cnw[n], p.cbias[o]);
    }
    if (tid < M * 32) {
        const int m = tid >> 5, pp = tid & 31;
        SF.mx[m][pp] = p.mx ? p.mx[((int64_t)h * M + m) * 64 + p0 + pp] : 1.f;
    }
    // state tile of this wave: headdim rows p0..p0+31, dstate columns 32 wave..
    s3_f32x16_t hacc;
    const int64_t hbase = bh * 64 * N;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int pp = p0 + 8 * (v >> 2) + 4 * half + (v & 3);
        hacc[v] = p.h0[hbase + pp * N + wave * 32 + r];
    }
#pragma unroll
    for (int v = 0; v < 16; ++v)
        S.h[0][8 * (v >> 2) + 4 * half + (v & 3)][wave * 32 + r] = __builtin_bit_cast(bf16_t, (__bf16)hacc[v]);

    const float dtb = p.dt_bias[h];
    const float Dv = p.Dh ? p.Dh[h] : 0.f;
    const bf16_t* projb = p.proj + (int64_t)b * p.proj_sb;
    const uint32_t rs = (uint32_t)p.proj_sl * 2;  // bytes per proj row (the host bounds (TS + 1) rows below 2^31)
    bf16_t* yhead = p.y + (int64_t)b * p.L * M * p.H * 64 + (int64_t)h * 64 + p0;
    const uint32_t y_rs = (uint32_t)p.H * 64 * 2;

    // ---- thread roles and their byte offsets within a chunk's proj rows
    // coefficients: fused position f = tid (< QF) of step f >> lgM
    const int cf_tl = (tid & (QF - 1)) >> lgM;
    const bool cf_first = (tid & (M - 1)) == 0;
    const uint32_t co_dt = (uint32_t)cf_tl * rs + (uint32_t)(p.o_dt + h) * 2;
    const uint32_t co_da = co_dt + (uint32_t)p.H * 2, co_lam = co_dt + (uint32_t)p.H * 4;
    // angles: a = tid / 4 over steps q JA .. q JA + JA - 1, q = tid % 4
    const int ang_a = tid >> 2, ang_q = tid & 3;
    const uint32_t ao = (uint32_t)(ang_q * JA) * rs + (uint32_t)(p.o_dt + 3 * p.H + min(ang_a, p.A - 1)) * 2;
    // B items: rows f0 = 2 (b_fp + 16 k) and f0 + 1 (ranks bm0, bm0 + 1 of one step), columns 8 b_nv..
    const int b_fp = tid >> 4, b_nv = tid & 15;
    const int bm0 = (2 * b_fp) & (M - 1);
    const uint32_t bo = (uint32_t)((2 * b_fp) >> lgM) * rs + (uint32_t)(p.o_b + (bm0 * p.G + g) * N + b_nv * 8) * 2;
    const uint32_t b_r2 = (uint32_t)p.G * N * 2;
    // C fragments: row i = 32 wave + r, columns 16 kn + 8 half .. (+8) for kn = 0..7
    const int c_i = wave * 32 + r, c_tl = c_i >> lgM, c_m = c_i & (M - 1);
    const uint32_t cofs = (uint32_t)c_tl * rs + (uint32_t)(p.o_c + (c_m * p.G + g) * N + 8 * half) * 2;

    // ---- register prefetch of one chunk's raw proj data
    uint2 xq[XPT];
    uint4 bq[BPT][2], cn[NK];
    uint32_t cq[5] = {0u, 0u, 0u, 0u, 0u};
    uint32_t rq[JA];
    // rows of chunk c and the step after it (scale's shift); zero past the end
    auto chunk_rsrc = [&](int c) {
        const int steps = min(TS + 1, p.L - c * TS);
        return buf_rsrc(projb + (int64_t)c * TS * p.proj_sl, (uint32_t)steps * rs);
    };
    auto fetch = [&](int c) {
        const __amdgpu_buffer_rsrc_t rp = chunk_rsrc(c);
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = tid + 256 * k;
            if (XI % 256 == 0 || item < XI)
                xq[k] = buf_ld8(rp, (uint32_t)(item >> 3) * rs + (uint32_t)(p.o_x + h * 64 + p0 + (item & 7) * 4) * 2);
        }
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            const uint32_t o = bo + (uint32_t)((32 * k) >> lgM) * rs;
            bq[k][0] = buf_ld16(rp, o);
            bq[k][1] = buf_ld16(rp, o + b_r2);
        }
        if (tid < QF) {
            cq[0] = buf_ld2(rp, co_dt);
            cq[1] = buf_ld2(rp, co_da);
            cq[2] = buf_ld2(rp, co_lam);
            cq[3] = buf_ld2(rp, co_dt + rs);
            cq[4] = buf_ld2(rp, co_lam + rs);
        }
#pragma unroll
        for (int j = 0; j < JA; ++j) rq[j] = buf_ld2(rp, ao + (uint32_t)j * rs);
    };
    auto fetch_c = [&](int c) {
        const __amdgpu_buffer_rsrc_t rp = chunk_rsrc(c);
#pragma unroll
        for (int kn = 0; kn < NK; ++kn) cn[kn] = buf_ld16(rp, cofs + 32 * kn);
    };
    fetch(0);
    fetch_c(0);
    float theta = ang_a < p.A ? p.ang[bh * p.A + ang_a] : 0.f;

    for (int c = 0; c < p.nch; ++c) {
        const int cur = c & 1;
        const int t0 = c * TS;
        // ---- A: coefficients of this thread's position; the block scan of da
        float daq = 0.f, scq = 0.f, gmq = 0.f;
        if (tid < QF) {
            const int t = t0 + cf_tl;
            float dt = 0.f;
            if (t < p.L) {
                dt = fminf(fmaxf(m3p_softplus(m3f_bf(cq[0]) + dtb), p.dt_lo), p.dt_hi);
                const float da = dt * -fmaxf(m3p_softplus(m3f_bf(cq[1])), p.a_floor);
                const float lam = 1.f / (1.f + __expf(-m3f_bf(cq[2])));
                float nxt = 0.f;
                if (t + 1 < p.L) {
                    const float dt1 = fminf(fmaxf(m3p_softplus(m3f_bf(cq[3]) + dtb), p.dt_lo), p.dt_hi);
                    const float lam1 = 1.f / (1.f + __expf(-m3f_bf(cq[4])));
                    nxt = (1.f - lam1) * dt1;
                }
                gmq = lam * dt;
                scq = gmq + nxt;
                daq = cf_first ? da : 0.f;  // da enters the cumulative sum once per step
            }
            if (cf_first) SF.dt[cf_tl] = dt;
        }
        const float loc = wave_incl_scan(daq * kLog2eS3);
        if (lane == 63) S.red[wave] = loc;
        if ((tid & 31) == 0 && tid < QF) S.anc[tid >> 5] = loc;
        __syncthreads();
        // ---- B: per-position tables; angles and their cos / sin
        const float cs_end = (S.red[0] + S.red[1]) + (S.red[2] + S.red[3]);
        if (tid < QF) {
            const int j = tid;
            float off = 0.f;
#pragma unroll
            for (int k = 0; k < 3; ++k)
                if (k < wave) off += S.red[k];
            const float csj = loc + off;
            S.cs2[j] = csj;
            S.st[j] = (float)(j >> lgM);
            S.sc[j] = scq;
            S.gm[j] = gmq;
            S.w[j] = scq * __builtin_amdgcn_exp2f(cs_end - csj);
#pragma unroll
            for (int it = 1; it < 4; ++it) {
                if (j < it * 32) {
                    float anchor = S.anc[it];
#pragma unroll
                    for (int k = 0; k < 3; ++k)
                        if (k < (it >> 1)) anchor += S.red[k];
                    S.f[it - 1][j] = scq * __builtin_amdgcn_exp2f(anchor - csj);
                }
            }
        }
        {
            float cum[JA];
            float run = 0.f;
#pragma unroll
            for (int j = 0; j < JA; ++j) {
                run += SF.dt[ang_q * JA + j] * (m3_tanh(m3f_bf(rq[j])) * p.span);
                cum[j] = run;
            }
            // exclusive prefix of the quarters' totals inside the quad (lanes 4 a .. 4 a + 3)
            const float q0 = m3_dpp<0x00>(run), q1 = m3_dpp<0x55>(run), q2 = m3_dpp<0xAA>(run);
            const float base = theta + ((ang_q >= 1 ? q0 : 0.f) + (ang_q >= 2 ? q1 : 0.f) + (ang_q >= 3 ? q2 : 0.f));
            const bool rot_on = ang_a < p.npair;
#pragma unroll
            for (int j = 0; j < JA; ++j) {
                const float th = m3p_wrap(base + cum[j]);
                SF.cs[ang_q * JA + j][ang_a] = rot_on ? __cosf(th) : 1.f;
                SF.sn[ang_q * JA + j][ang_a] = rot_on ? __sinf(th) : 0.f;
            }
            // the chunk's last angle (quarter 3's), carried wrapped
            theta = m3p_wrap(m3_dpp<0xFF>(base + cum[JA - 1]));
        }
        __syncthreads();
        // ---- C: B rows to LDS; v^T and w-scaled v^T; this wave's C fragments
        {
            const int kb = (b_nv & 7) * 8;  // pair index of this thread's first column
            const float sgn = b_nv < 8 ? -1.f : 1.f;
            float bw[8], bb0[8], bb1[8];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float4 u0 = *(const float4*)&SF.bwb[bm0][b_nv * 8 + e];
                const float4 u1 = *(const float4*)&SF.bwb[bm0 + 1][b_nv * 8 + e];
                bw[e] = u0.x; bb0[e] = u0.y; bw[e + 1] = u0.z; bb0[e + 1] = u0.w;
                bb1[e] = u1.y; bb1[e + 1] = u1.w;
            }
#pragma unroll
            for (int k = 0; k < BPT; ++k) {
                const int f0 = 2 * (b_fp + 16 * k), tl = f0 >> lgM;
                float y0[8], y1[8];
                const uint32_t a0[4] = {bq[k][0].x, bq[k][0].y, bq[k][0].z, bq[k][0].w};
                const uint32_t a1[4] = {bq[k][1].x, bq[k][1].y, bq[k][1].z, bq[k][1].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y0[2 * e] = s3_lo(a0[e]); y0[2 * e + 1] = s3_hi(a0[e]);
                    y1[2 * e] = s3_lo(a1[e]); y1[2 * e + 1] = s3_hi(a1[e]);
                }
                float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    ss0 += y0[e] * y0[e];
                    ss1 += y1[e] * y1[e];
                }
                ss0 = m3_group_sum<16>(ss0);
                ss1 = m3_group_sum<16>(ss1);
                const float rms0 = 1.f / sqrtf(ss0 / (float)N + kDivEpsF32);
                const float rms1 = 1.f / sqrtf(ss1 / (float)N + kDivEpsF32);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    y0[e] = (y0[e] * rms0) * bw[e] + bb0[e];
                    y1[e] = (y1[e] * rms1) * bw[e] + bb1[e];
                }
                float o0[8], o1[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    o0[e] = m3_xor<8>(y0[e]);
                    o1[e] = m3_xor<8>(y1[e]);
                }
                const float4 c0 = *(const float4*)&SF.cs[tl][kb], c1 = *(const float4*)&SF.cs[tl][kb + 4];
                const float4 s0 = *(const float4*)&SF.sn[tl][kb], s1 = *(const float4*)&SF.sn[tl][kb + 4];
                const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    y0[e] = cv[e] * y0[e] + (sgn * sv[e]) * o0[e];
                    y1[e] = cv[e] * y1[e] + (sgn * sv[e]) * o1[e];
                }
                *(uint4*)&S.B[f0][b_nv * 8] = make_uint4(pack_bf16x2(y0[0], y0[1]), pack_bf16x2(y0[2], y0[3]),
                                                        pack_bf16x2(y0[4], y0[5]), pack_bf16x2(y0[6], y0[7]));
                *(uint4*)&S.B[f0 + 1][b_nv * 8] = make_uint4(pack_bf16x2(y1[0], y1[1]), pack_bf16x2(y1[2], y1[3]),
                                                            pack_bf16x2(y1[4], y1[5]), pack_bf16x2(y1[6], y1[7]));
                // the cache tail: the last step's rotated B (f32)
                if (ph == 0 && t0 + tl == p.L - 1) {
                    float* k0 = p.kst + (((int64_t)b * M + bm0) * p.H + h) * N + b_nv * 8;
                    float* k1 = p.kst + (((int64_t)b * M + bm0 + 1) * p.H + h) * N + b_nv * 8;
                    *(float4*)k0 = make_float4(y0[0], y0[1], y0[2], y0[3]);
                    *(float4*)(k0 + 4) = make_float4(y0[4], y0[5], y0[6], y0[7]);
                    *(float4*)k1 = make_float4(y1[0], y1[1], y1[2], y1[3]);
                    *(float4*)(k1 + 4) = make_float4(y1[4], y1[5], y1[6], y1[7]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = tid + 256 * k;
            if (XI % 256 == 0 || item < XI) {
                const int tl = item >> 3, pv = item & 7;
                const float xv[4] = {s3_lo(xq[k].x), s3_hi(xq[k].x), s3_lo(xq[k].y), s3_hi(xq[k].y)};
                if (t0 + tl == p.L - 1)  // the cache tail: the last step's x
                    *(float4*)(p.vst + bh * 64 + p0 + pv * 4) = make_float4(xv[0], xv[1], xv[2], xv[3]);
                float vt[4][M], vw[4][M];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float wf = S.w[tl * M + m];
                    const float4 mv = *(const float4*)&SF.mx[m][pv * 4];
                    const float mxa[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float vb = (float)(__bf16)(xv[e] * mxa[e]);  // v as the SSD seam holds it (bf16)
                        vt[e][m] = vb;
                        vw[e][m] = vb * wf;
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    m3f_st<M>(&S.xT[pv * 4 + e][tl * M], vt[e]);
                    m3f_st<M>(&S.xTw[pv * 4 + e][tl * M], vw[e]);
                }
            }
        }
        s3_bf16x8_t cfr[NK];
        {
            float cv[NK][8];
#pragma unroll
            for (int kn = 0; kn < NK; ++kn) {
                const uint32_t a[4] = {cn[kn].x, cn[kn].y, cn[kn].z, cn[kn].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cv[kn][2 * e] = s3_lo(a[e]);
                    cv[kn][2 * e + 1] = s3_hi(a[e]);
                }
            }
            float ss = 0.f;
#pragma unroll
            for (int kn = 0; kn < NK; ++kn)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += cv[kn][e] * cv[kn][e];
            ss += __shfl_xor(ss, 32, 64);  // the row's other 64 columns
            const float rms = 1.f / sqrtf(ss / (float)N + kDivEpsF32);
#pragma unroll
            for (int kn = 0; kn < NK / 2; ++kn) {
                const int n0 = 16 * kn + 8 * half;  // columns n0 .. n0 + 7 and their partners n0 + 64 ..
                float lo[8], hi[8];
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float4 u = *(const float4*)&SF.cwb[c_m][n0 + e];
                    const float4 v = *(const float4*)&SF.cwb[c_m][n0 + 64 + e];
                    lo[e] = (cv[kn][e] * rms) * u.x + u.y;
                    lo[e + 1] = (cv[kn][e + 1] * rms) * u.z + u.w;
                    hi[e] = (cv[kn + 4][e] * rms) * v.x + v.y;
                    hi[e + 1] = (cv[kn + 4][e + 1] * rms) * v.z + v.w;
                }
                const float4 c0 = *(const float4*)&SF.cs[c_tl][n0], c1 = *(const float4*)&SF.cs[c_tl][n0 + 4];
                const float4 s0 = *(const float4*)&SF.sn[c_tl][n0], s1 = *(const float4*)&SF.sn[c_tl][n0 + 4];
                const float ca[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                const float sa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    cfr[kn][e] = (__bf16)(ca[e] * lo[e] + (-sa[e]) * hi[e]);
                    cfr[kn + 4][e] = (__bf16)(ca[e] * hi[e] + sa[e] * lo[e]);
                }
            }
        }
        // ---- the next chunk's loads land during this chunk's MFMA work
        if (c + 1 < p.nch) fetch(c + 1);
        __syncthreads();
        // ---- D: state h <- exp(cs_end) h + sum_j (w_j v^T[p][j]) B[j][n], n tile = wave
        {
            const float dec = __builtin_amdgcn_exp2f(cs_end);
#pragma unroll
            for (int v = 0; v < 16; ++v) hacc[v] *= dec;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int j0 = ks * 16 + 8 * half;
                const s3_bf16x8_t a = *(const s3_bf16x8_t*)&S.xTw[r][j0];
                s3_bf16x8_t bo8;
#pragma unroll
                for (int e = 0; e < 8; ++e) bo8[e] = __builtin_bit_cast(__bf16, S.B[j0 + e][wave * 32 + r]);
                hacc = s3_mfma(a, bo8, hacc);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
                S.h[cur ^ 1][8 * (v >> 2) + 4 * half + (v & 3)][wave * 32 + r] =
                    __builtin_bit_cast(bf16_t, (__bf16)hacc[v]);
        }
        // ---- y for output tile = wave, plus D v
        {
            s3_f32x16_t yacc;
            switch (wave) {
                case 0: ssd3_y_tile<QF, 0>(S, cfr, cur, r, half, yacc); break;
                case 1: ssd3_y_tile<QF, 1>(S, cfr, cur, r, half, yacc); break;
                case 2: ssd3_y_tile<QF, 2>(S, cfr, cur, r, half, yacc); break;
                default: ssd3_y_tile<QF, 3>(S, cfr, cur, r, half, yacc); break;
            }
            if (p.Dh) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int pp = 8 * (v >> 2) + 4 * half + (v & 3);
                    yacc[v] += Dv * bf16_to_f32(S.xT[pp][wave * 32 + r]);
                }
            }
            // stage the 32 (position) x 32 (p) tile: lane holds y[i][p = 8(v/4) + 4 half + v%4]
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const s3_bf16x4_t q = {(__bf16)yacc[4 * gq], (__bf16)yacc[4 * gq + 1], (__bf16)yacc[4 * gq + 2],
                                       (__bf16)yacc[4 * gq + 3]};
                *(s3_bf16x4_t*)&S.y[wave][r][8 * gq + 4 * half] = q;
            }
            __builtin_amdgcn_wave_barrier();  // LDS ops of one wave complete in order
            if (c + 1 < p.nch) fetch_c(c + 1);
            // 32 rows x 64 bytes: 4 lanes per row, 16 rows per instruction
            const int rows = min(QF, (p.L - t0) * M);
            const __amdgpu_buffer_rsrc_t ry = buf_rsrc(yhead + (int64_t)t0 * M * p.H * 64, (uint32_t)rows * y_rs);
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int row = q * 16 + (lane >> 2), ch = lane & 3;
                const uint4 val = *(const uint4*)&S.y[wave][row][ch * 8];
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(decltype(__builtin_amdgcn_raw_buffer_load_b128(ry, 0, 0, 0)), val), ry,
                    (uint32_t)(wave * 32 + row) * y_rs + ch * 16, 0, 0);
            }
        }
        __syncthreads();  // LDS reads of this chunk done before the next commit
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int pp = p0 + 8 * (v >> 2) + 4 * half + (v & 3);
        p.hT[hbase + pp * N + wave * 32 + r] = hacc[v];
    }
    if (ph == 0 && ang_q == 0 && ang_a < p.A) p.ang_out[bh * p.A + ang_a] = theta;
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
    *ok = p.proj_bf16 && p.P == 64 && p.N == 128 && (M == 2 || M == 4 || M == 8) && al16(p.proj) &&
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
    const dim3 grid(fp.nb * fp.H * 2), block(256);
    switch (pp.M) {
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
