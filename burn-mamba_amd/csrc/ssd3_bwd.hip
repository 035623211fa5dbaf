// Mamba-3 SSD backward (recompute form), gfx950: gradients of the single-SSD
// forward (ssd3.hip / ssd3_mfma.hip) with respect to v, da, B, C, gamma, scale
// and the initial state, from dy and d(final state).  With gamma = scale = 1
// (NULL) it is the double-SSD seam's backward, whose forward is the single one
// with unit weights.
//
// Reference: the Autodiff arms of Mamba3SingleSsdBackendExt::single_ssd_serial_
// recalculated (src/mamba3/single_ssd/ssd/serial_recalculated/backward.rs:27-299,
// gradient math combined_backward.rs:74-536) and of Mamba3DoubleSsdBackendExt::
// double_ssd_serial_recalculated (double_ssd/ssd/serial_recalculated/
// backward.rs:27-275, combined_backward.rs:98-542).
//
// The forward per (batch, head) and step t, K_t = sum_m v[t,m] B[t,m]^T:
//   S_t = exp(da_t) h_{t-1},  h_t = S_t + scale_t K_t,
//   y[t,mo] = S_t C[t,mo] + gamma_t sum_mi (C[t,mo].B[t,mi]) v[t,mi].
// Chunks of 32 fused positions j = (step t, rank m), j = t M + m, i.e. 32 / M
// steps.  With cs the within-chunk cumulative sum of da over steps, a_t =
// exp(cs_end - cs_t), b_t = exp(cs_t), h_c the state entering the chunk, g the
// gradient of the state leaving it, and the fused weight
//   W[k][i] = exp(cs_t(k) - cs_t(i)) scale_t(i)   for t(k) > t(i),
//             gamma_t(k)                          for t(k) = t(i),   0 otherwise,
// every gradient is written without a P x N matrix per position:
//   dv_j = scale_t a_t g B_j + sum_k W[k][j] (C_k.B_j) dy_k
//   dB_j = scale_t a_t g^T v_j + sum_k W[k][j] (dy_k.v_j) C_k
//   dC_k = b_t h_c^T dy_k + sum_i W[k][i] (dy_k.v_i) B_i
//   dscale_t = a_t sum_{j in t} v_j.g B_j + sum_{i in t} sum_{t(k) > t} e_{t(k) t} (C_k.B_i)(dy_k.v_i)
//   dgamma_t = sum_{k, i in t} (C_k.B_i)(dy_k.v_i)
//   dda_t = a_t b_t <g, h_c> + a_t s1_t + b_t s2_t + sum_{t' < t} (colm_t' - rowm_t')
// with s1_t = sum_{t'<t} e_{t t'} scale_t' sum_{j in t'} v_j.g B_j, s2_t =
// sum_{t''>=t} e_{t'' t} sum_{k in t''} dy_k.h_c C_k, and colm / rowm the
// column / row sums over steps of M_ki = W[k][i] (C_k.B_i)(dy_k.v_i) restricted
// to t(k) > t(i).  The gradient entering the previous chunk is
// exp(cs_end) g + sum_k b_t(k) dy_k C_k^T.  f32 throughout.
#include <algorithm>

#include "bwd_core.h"
#include "common.h"

namespace mamba {

constexpr int kB3F = 32;     // fused positions per chunk
constexpr int kB3T = 256;    // threads per workgroup (SIMT kernels)

struct Ssd3BwdParams {
    int nb, L, M, H, P, G, N, nch, QS;   // QS = steps per chunk = 32 / M
    const float* v; int64_t v_sb, v_sl, v_sm, v_sh;
    const float* da; int64_t da_sb, da_sl, da_sh;
    const float* gam; int64_t gam_sb, gam_sl, gam_sh;   // NULL: 1
    const float* scl; int64_t scl_sb, scl_sl, scl_sh;   // NULL: 1
    const float* B; int64_t B_sb, B_sl, B_sm, B_sg;
    const float* C; int64_t C_sb, C_sl, C_sm, C_sg;
    const float* h0;
    const float* dy; int64_t dy_sb, dy_sl, dy_sm, dy_sh;
    const float* dfin;
    float* dv; float* dda; float* dgam; float* dscl;     // dgam / dscl NULL without the weights
    float* dBh; float* dCh;                               // [b, l, m, h, n] per head
    float* dh0;
    float* hs;                                            // [b, h, nch, P, N] chunk-entry states
    float* dvp;                                           // [2][b, l, m, h, p] partial dv (half-dstate kernel)
    float* sp;                                            // [3][2][b, l, h] partial dda, dscale, dgamma
};

// Per-step scalars of chunk c for threads 0..QS-1: da, gamma, scale (0 past the end).
__device__ __forceinline__ void b3_step_scalars(const Ssd3BwdParams& p, int b, int h, int c, float* das, float* gms,
                                                float* scs) {
    const int t = threadIdx.x;
    if (t < p.QS) {
        const int ts = c * p.QS + t;
        const bool ok = ts < p.L;
        das[t] = ok ? p.da[(int64_t)b * p.da_sb + (int64_t)ts * p.da_sl + (int64_t)h * p.da_sh] : 0.f;
        gms[t] = ok ? (p.gam ? p.gam[(int64_t)b * p.gam_sb + (int64_t)ts * p.gam_sl + (int64_t)h * p.gam_sh] : 1.f) : 0.f;
        scs[t] = ok ? (p.scl ? p.scl[(int64_t)b * p.scl_sb + (int64_t)ts * p.scl_sl + (int64_t)h * p.scl_sh] : 1.f) : 0.f;
    }
}

// within-chunk cumulative sum of da over steps (thread 0) and its factors
__device__ __forceinline__ void b3_cumsum(int QS, const float* das, float* cs, float* av, float* bv) {
    if (threadIdx.x == 0) {
        float run = 0.f;
        for (int t = 0; t < QS; ++t) {
            run += das[t];
            cs[t] = run;
        }
        for (int t = 0; t < QS; ++t) {
            av[t] = __expf(run - cs[t]);
            bv[t] = __expf(cs[t]);
        }
    }
}

// Fused rows of chunk c into LDS: W-wide rows of a [b, l, m, (h|g), W] tensor;
// rows past the sequence end are zero.
__device__ __forceinline__ void b3_rows(float* dst, const float* base, int64_t s_l, int64_t s_m, int c, const Ssd3BwdParams& p,
                                        int W) {
    for (int e = threadIdx.x; e < kB3F * W; e += kB3T) {
        const int j = e / W, w = e - j * W;
        const int t = j / p.M, m = j - t * p.M;
        const int ts = c * p.QS + t;
        dst[e] = ts < p.L ? base[(int64_t)ts * s_l + (int64_t)m * s_m + w] : 0.f;
    }
}

// Chunk-entry states (the forward's K3 + K4).  One workgroup per (batch, head).
// Dynamic LDS: [P N] state + [32][P] v + [32][N] B.
__global__ __launch_bounds__(kB3T) void ssd3_bwd_states(Ssd3BwdParams p) {
    extern __shared__ float s_dyn[];
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H, g = h / (p.H / p.G);
    const int P = p.P, N = p.N, PN = P * N;
    float* hst = s_dyn;
    float* vs = hst + PN;
    float* Bs = vs + kB3F * P;
    __shared__ float das[kB3F], gms[kB3F], scs[kB3F], cs[kB3F], av[kB3F], bv[kB3F];
    const int64_t bh = (int64_t)b * p.H + h;
    for (int e = threadIdx.x; e < PN; e += kB3T) hst[e] = p.h0 ? p.h0[bh * PN + e] : 0.f;
    const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    __syncthreads();
    for (int c = 0; c < p.nch; ++c) {
        float* dst = p.hs + (bh * p.nch + c) * PN;
        for (int e = threadIdx.x; e < PN; e += kB3T) dst[e] = hst[e];
        b3_rows(vs, vb, p.v_sl, p.v_sm, c, p, P);
        b3_rows(Bs, Bb, p.B_sl, p.B_sm, c, p, N);
        b3_step_scalars(p, b, h, c, das, gms, scs);
        __syncthreads();
        b3_cumsum(p.QS, das, cs, av, bv);
        __syncthreads();
        const float dec = __expf(cs[p.QS - 1]);
        for (int e = threadIdx.x; e < PN; e += kB3T) {
            const int pp = e / N, n = e - pp * N;
            float acc = dec * hst[e];
            for (int j = 0; j < kB3F; ++j) {
                const int t = j / p.M;
                acc += (av[t] * scs[t]) * vs[j * P + pp] * Bs[j * N + n];
            }
            hst[e] = acc;
        }
        __syncthreads();
    }
}

__device__ __forceinline__ float b3_block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// The reverse chunk loop (SIMT).  One workgroup per (batch, head).  Dynamic
// LDS: g, h_c [P N]; v, dy, u [32][P]; B, C [32][N]; W, CB, DX [32][32].
__global__ __launch_bounds__(kB3T) void ssd3_bwd_chunks(Ssd3BwdParams p) {
    extern __shared__ float s_dyn[];
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H, g = h / (p.H / p.G);
    const int P = p.P, N = p.N, PN = P * N, M = p.M, QS = p.QS;
    constexpr int F = kB3F;
    float* gs = s_dyn;
    float* hc = gs + PN;
    float* vs = hc + PN;
    float* dys = vs + F * P;
    float* us = dys + F * P;
    float* Bs = us + F * P;
    float* Cs = Bs + F * N;
    float* Ws = Cs + F * N;
    float* CBs = Ws + F * F;
    float* DXs = CBs + F * F;
    __shared__ float das[F], gms[F], scs[F], cs[F], av[F], bv[F];
    __shared__ float xuf[F], qhf[F], xus[F], qhs[F], xg2s[F], colm[F], rowm[F], red[4];
    const int64_t bh = (int64_t)b * p.H + h;
    const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
    const float* yb = p.dy + (int64_t)b * p.dy_sb + (int64_t)h * p.dy_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    const float* Cb = p.C + (int64_t)b * p.C_sb + (int64_t)g * p.C_sg;
    const int tid = threadIdx.x;
    for (int e = tid; e < PN; e += kB3T) gs[e] = p.dfin ? p.dfin[bh * PN + e] : 0.f;
    for (int c = p.nch - 1; c >= 0; --c) {
        __syncthreads();  // the previous chunk's readers of the chunk buffers are done
        const float* src = p.hs + (bh * p.nch + c) * PN;
        for (int e = tid; e < PN; e += kB3T) hc[e] = src[e];
        b3_rows(vs, vb, p.v_sl, p.v_sm, c, p, P);
        b3_rows(dys, yb, p.dy_sl, p.dy_sm, c, p, P);
        b3_rows(Bs, Bb, p.B_sl, p.B_sm, c, p, N);
        b3_rows(Cs, Cb, p.C_sl, p.C_sm, c, p, N);
        b3_step_scalars(p, b, h, c, das, gms, scs);
        __syncthreads();
        b3_cumsum(QS, das, cs, av, bv);
        float ghp = 0.f;
        for (int e = tid; e < PN; e += kB3T) ghp += gs[e] * hc[e];
        const float ghc = b3_block_sum(ghp, red);  // (its barriers also publish cs / av / bv)
        // fused Q x Q products and weights; u_j = g B_j
        for (int e = tid; e < F * F; e += kB3T) {
            const int k = e / F, i = e - k * F;
            const int tk = k / M, ti = i / M;
            float cb = 0.f, dx = 0.f;
            for (int n = 0; n < N; ++n) cb += Cs[k * N + n] * Bs[i * N + n];
            for (int pp = 0; pp < P; ++pp) dx += dys[k * P + pp] * vs[i * P + pp];
            CBs[e] = cb;
            DXs[e] = dx;
            Ws[e] = tk > ti ? __expf(cs[tk] - cs[ti]) * scs[ti] : (tk == ti ? gms[tk] : 0.f);
        }
        for (int e = tid; e < F * P; e += kB3T) {
            const int j = e / P, pp = e - j * P;
            float acc = 0.f;
            for (int n = 0; n < N; ++n) acc += gs[pp * N + n] * Bs[j * N + n];
            us[e] = acc;
        }
        // qh_k = dy_k^T h_c C_k: 8 threads per k
        {
            const int k = tid >> 3, part = tid & 7;
            float acc = 0.f;
            for (int pp = part; pp < P; pp += 8) {
                float w = 0.f;
                for (int n = 0; n < N; ++n) w += hc[pp * N + n] * Cs[k * N + n];
                acc += dys[k * P + pp] * w;
            }
            acc += __shfl_xor(acc, 1, 64);
            acc += __shfl_xor(acc, 2, 64);
            acc += __shfl_xor(acc, 4, 64);
            if (part == 0) qhf[k] = acc;
        }
        __syncthreads();
        if (tid < F) {
            float a = 0.f;
            for (int pp = 0; pp < P; ++pp) a += vs[tid * P + pp] * us[tid * P + pp];
            xuf[tid] = a;
        }
        __syncthreads();
        // per step: the sums over the step's ranks
        if (tid < QS) {
            const int t = tid;
            float xu = 0.f, qh = 0.f, xg2 = 0.f, rm = 0.f;
            for (int m = 0; m < M; ++m) {
                xu += xuf[t * M + m];
                qh += qhf[t * M + m];
            }
            for (int i = t * M; i < t * M + M; ++i)
                for (int k = (t + 1) * M; k < F; ++k) xg2 += __expf(cs[k / M] - cs[t]) * CBs[k * F + i] * DXs[k * F + i];
            for (int k = t * M; k < t * M + M; ++k)
                for (int i = 0; i < t * M; ++i) rm += Ws[k * F + i] * CBs[k * F + i] * DXs[k * F + i];
            xus[t] = xu;
            qhs[t] = qh;
            xg2s[t] = xg2;
            colm[t] = scs[t] * xg2;
            rowm[t] = rm;
        }
        __syncthreads();
        if (tid < QS) {
            const int t = tid, ts = c * QS + t;
            float s1 = 0.f, s2 = 0.f, pre = 0.f, dg = 0.f;
            for (int tt = 0; tt < t; ++tt) {
                s1 += __expf(cs[t] - cs[tt]) * scs[tt] * xus[tt];
                pre += colm[tt] - rowm[tt];
            }
            for (int tt = t; tt < QS; ++tt) s2 += __expf(cs[tt] - cs[t]) * qhs[tt];
            for (int k = t * M; k < t * M + M; ++k)
                for (int i = t * M; i < t * M + M; ++i) dg += CBs[k * F + i] * DXs[k * F + i];
            if (ts < p.L) {
                const int64_t o = (int64_t)b * p.L * p.H + (int64_t)ts * p.H + h;
                p.dda[o] = av[t] * bv[t] * ghc + av[t] * s1 + bv[t] * s2 + pre;
                if (p.dscl) p.dscl[o] = av[t] * xus[t] + xg2s[t];
                if (p.dgam) p.dgam[o] = dg;
            }
        }
        // dv_j = scale_t a_t g B_j + sum_k W[k][j] (C_k.B_j) dy_k
        for (int e = tid; e < F * P; e += kB3T) {
            const int j = e / P, pp = e - j * P, t = j / M, m = j - t * M;
            const int ts = c * QS + t;
            if (ts >= p.L) continue;
            float acc = scs[t] * av[t] * us[e];
            for (int k = 0; k < F; ++k) acc += Ws[k * F + j] * CBs[k * F + j] * dys[k * P + pp];
            p.dv[((((int64_t)b * p.L + ts) * M + m) * p.H + h) * P + pp] = acc;
        }
        // dB_j = scale_t a_t g^T v_j + sum_k W[k][j] (dy_k.v_j) C_k; dC_k = b_t h_c^T dy_k + sum_i W[k][i] (dy_k.v_i) B_i
        for (int e = tid; e < F * N; e += kB3T) {
            const int j = e / N, n = e - j * N, t = j / M, m = j - t * M;
            const int ts = c * QS + t;
            if (ts >= p.L) continue;
            float gx = 0.f, hd = 0.f;
            for (int pp = 0; pp < P; ++pp) {
                gx += gs[pp * N + n] * vs[j * P + pp];
                hd += hc[pp * N + n] * dys[j * P + pp];
            }
            float sb = scs[t] * av[t] * gx, sc = bv[t] * hd;
            for (int k = 0; k < F; ++k) sb += Ws[k * F + j] * DXs[k * F + j] * Cs[k * N + n];
            for (int i = 0; i < F; ++i) sc += Ws[j * F + i] * DXs[j * F + i] * Bs[i * N + n];
            const int64_t o = ((((int64_t)b * p.L + ts) * M + m) * p.H + h) * N + n;
            p.dBh[o] = sb;
            p.dCh[o] = sc;
        }
        __syncthreads();  // every reader of g for this chunk is done
        const float dec = __expf(cs[QS - 1]);
        for (int e = tid; e < PN; e += kB3T) {
            const int pp = e / N, n = e - pp * N;
            float acc = dec * gs[e];
            for (int k = 0; k < F; ++k) acc += bv[k / M] * dys[k * P + pp] * Cs[k * N + n];
            gs[e] = acc;
        }
    }
    __syncthreads();
    for (int e = tid; e < PN; e += kB3T) p.dh0[bh * PN + e] = gs[e];
}

// dB / dC summed over the heads of each group (in head order) when ngroups < nheads.
__global__ __launch_bounds__(256) void ssd3_bwd_finish(Ssd3BwdParams p, float* dB, float* dC) {
    const int rep = p.H / p.G;
    const int64_t total = (int64_t)p.nb * p.L * p.M * p.G * p.N;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int n = (int)(e % p.N);
        const int64_t r = e / p.N;
        const int gg = (int)(r % p.G);
        const int64_t blm = r / p.G;
        float sb = 0.f, sc = 0.f;
        for (int k = 0; k < rep; ++k) {
            const int64_t o = (blm * p.H + (int64_t)gg * rep + k) * p.N + n;
            sb += p.dBh[o];
            sc += p.dCh[o];
        }
        dB[e] = sb;
        dC[e] = sc;
    }
}

// ---------------------------------------------------------------------------
// MFMA path for headdim 64 x dstate 128 (the config-4 head shape): the Mamba-2
// backward's f32 MFMA structure (bwd_core.h) on 32 fused rows per chunk, split
// over the two halves of dstate.  The per-step scalars are expanded over the
// step's M rows in LDS.

__device__ __forceinline__ int b3_lg(int M) { return 31 - __builtin_clz(M); }

// The reverse chunk loop over one half of dstate: two 512-thread workgroups
// per (batch, head), 69 KB of LDS each (every CU is busy at config 4's 128
// heads x batch rows).  The state columns split exactly: g, h_c, dB, dC and
// d(initial state) of a half are the half's own.  Sums over dstate (C.B,
// g B_j, C.h_c^T dy, <g, h_c>) are partial, and every gradient linear in them
// (dv, dda, dscale, dgamma) is written as one partial plane per half, summed
// in a fixed order by ssd3_bwd_half_finish.  Eight waves, 32 MFMAs each in
// phase 1 (waves w and w + 4 share a SIMD):
//   phase 1  w0, w1: g B_j (one 32-row half of p each, K = the half's 64 columns)
//            w2, w3: g^T v_j; w6, w7: h_c^T dy_j (one 32-column quarter each,
//            h_c's columns in registers); w4: C.B over the half; w5: dy.v
//   phase 2  w0, w1: dv; w2, w3: dB; w6, w7: dC; w4, w5: the update of g (two
//            tiles each); w3: the per-step scalars.
struct B3HalfLds {
    float g[kFP * kSX];      // [p][n] this half's columns of the state gradient
    float v[32 * kSX];       // [j][p]
    float dy[32 * kSX];      // [j][p]
    float B[32 * kSX];       // [j][n] this half's columns
    float C[32 * kSX];       // [j][n]
    float E1[32 * kSQ];      // [k][i] C_k . B_i over the half, then W o that
    float DX[32 * kSQ];      // [k][i] dy_k . v_i
    float E2[32 * kSQ];      // [k][i] W[k][i] dy_k . v_i
    float E3T[32 * kSQ];     // [i][k] W[k][i] dy_k . v_i
    float cs[32], av[32], bv[32], sc[32], gm[32];
    float xu[2][32];         // v_j . g B_j (this half of dstate), per 32-row half of p
    float qh[2][32];         // C_k . h_c^T dy_k, per 32-column quarter
    float ghc[2];
    float cpart[8][32];      // per-wave column sums of e (C.B)(dy.v) over later steps
    float rrow[32], rdg[32];
};

// One chunk's fused rows (v, dy full; B, C this half) and step scalars.
struct B3HalfRows {
    float4 v, dy, B, C;
    float da, gm, sc;
};

__device__ __forceinline__ void b3h_fetch(const Ssd3BwdParams& p, const float* vb, const float* yb, const float* Bb,
                                          const float* Cb, int b, int h, int c, int tid, int lg, int ns,
                                          B3HalfRows& f) {
    const int t0 = c * p.QS, mk = p.M - 1;
    const int j = tid >> 4, cx = (tid & 15) * 4;  // row j, a float4 of 64 columns
    const float4 z = {0.f, 0.f, 0.f, 0.f};
    const int t = t0 + (j >> lg), m = j & mk;
    const int64_t ot = (int64_t)min(t, p.L - 1);
    const float4 a = *reinterpret_cast<const float4*>(vb + ot * p.v_sl + (int64_t)m * p.v_sm + cx);
    const float4 y = *reinterpret_cast<const float4*>(yb + ot * p.dy_sl + (int64_t)m * p.dy_sm + cx);
    const float4 bb = *reinterpret_cast<const float4*>(Bb + ot * p.B_sl + (int64_t)m * p.B_sm + 64 * ns + cx);
    const float4 cc = *reinterpret_cast<const float4*>(Cb + ot * p.C_sl + (int64_t)m * p.C_sm + 64 * ns + cx);
    const int tt = t0 + ((tid & 31) >> lg);
    const int64_t os = (int64_t)min(tt, p.L - 1);
    const float da = p.da[(int64_t)b * p.da_sb + os * p.da_sl + (int64_t)h * p.da_sh];
    const float gm = p.gam ? p.gam[(int64_t)b * p.gam_sb + os * p.gam_sl + (int64_t)h * p.gam_sh] : 1.f;
    const float sc = p.scl ? p.scl[(int64_t)b * p.scl_sb + os * p.scl_sl + (int64_t)h * p.scl_sh] : 1.f;
    f.v = t < p.L ? a : z;
    f.dy = t < p.L ? y : z;
    f.B = t < p.L ? bb : z;
    f.C = t < p.L ? cc : z;
    f.da = tt < p.L ? da : 0.f;
    f.gm = tt < p.L ? gm : 0.f;
    f.sc = tt < p.L ? sc : 0.f;
}

__device__ __forceinline__ void b3h_commit(B3HalfLds& S, const B3HalfRows& f, int tid, int lg) {
    const int o = (tid >> 4) * kSX + (tid & 15) * 4;
    bwd_put4(&S.v[o], f.v);
    bwd_put4(&S.dy[o], f.dy);
    bwd_put4(&S.B[o], f.B);
    bwd_put4(&S.C[o], f.C);
    if (tid < 64) {
        const int lane = tid;
        const bool first = (lane & ((1 << lg) - 1)) == 0;
        const float cs = wave_incl_scan(lane < 32 && first ? f.da : 0.f);
        const float tot = __shfl(cs, 31, 64);
        if (lane < 32) {
            S.cs[lane] = cs;
            S.av[lane] = __expf(tot - cs);
            S.bv[lane] = __expf(cs);
            S.sc[lane] = f.sc;
            S.gm[lane] = f.gm;
        }
    }
}

// WPE = 1 gives the kernel 162 registers (one workgroup per CU); WPE = 4 holds
// it to 128 (a few spills) so that two workgroups share a CU, which pays once
// the grid has at least two workgroups per CU (21 % at batch 8 of config 4).
template <int WPE>
__global__ __launch_bounds__(512, WPE) void ssd3_bwd_chunks_half(Ssd3BwdParams p) {
    __shared__ B3HalfLds S;
    const int tid = threadIdx.x, wv = wave_id(), lane = tid & 63, i32 = lane & 31, hf = lane >> 5;
    const int ns = blockIdx.x & 1;
    const int b = (blockIdx.x >> 1) / p.H, h = (blockIdx.x >> 1) % p.H, grp = h / (p.H / p.G);
    const int lg = b3_lg(p.M), QS = p.QS;
    const int64_t bh = (int64_t)b * p.H + h;
    const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
    const float* yb = p.dy + (int64_t)b * p.dy_sb + (int64_t)h * p.dy_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)grp * p.B_sg;
    const float* Cb = p.C + (int64_t)b * p.C_sb + (int64_t)grp * p.C_sg;
    const int64_t nbl = (int64_t)p.nb * p.L;
    const int tq = wv & 1;  // 32-column quarter of waves 2, 3, 6, 7 within the half
    // h_c columns of waves 6-7: hreg[m] = h_c[2 m + hf][64 ns + 32 tq + i32]
    float hreg[32];
    auto fetch_h = [&](int c, float (&dst)[32]) {
        const float* src = p.hs + (bh * p.nch + c) * (kFP * kFN) + hf * kFN + 64 * ns + 32 * tq + i32;
#pragma unroll
        for (int m = 0; m < 32; ++m) dst[m] = src[m * 2 * kFN];
    };
    for (int e = tid; e < kFP * 64; e += 512)
        S.g[(e >> 6) * kSX + (e & 63)] = p.dfin ? p.dfin[bh * (kFP * kFN) + (e >> 6) * kFN + 64 * ns + (e & 63)] : 0.f;
    B3HalfRows pre;
    b3h_fetch(p, vb, yb, Bb, Cb, b, h, p.nch - 1, tid, lg, ns, pre);
    if (wv >= 6) fetch_h(p.nch - 1, hreg);
    b3h_commit(S, pre, tid, lg);
    __syncthreads();
    for (int c = p.nch - 1; c >= 0; --c) {
        const int t0 = c * QS;
        const int cn = c > 0 ? c - 1 : 0;
        int tid = threadIdx.x;  // opaque per chunk: keeps the LDS addresses in the loop
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, i32 = lane & 31, hf = lane >> 5;
        b3h_fetch(p, vb, yb, Bb, Cb, b, h, cn, tid, lg, ns, pre);
        // ---- phase 1: 32 MFMAs on every wave
        bwd_f32x16 acc = {};
        if (wv < 2) {  // u = g B_j for p rows 32 wv .., K = the half's 64 columns
            const float* Ap = S.B + i32 * kSX + hf;
            const float* Bp = S.g + (32 * wv + i32) * kSX + hf;
#pragma unroll 16
            for (int n0 = 0; n0 < 64; n0 += 2) acc = bwd_mfma(Ap[n0], Bp[n0], acc);
        } else if (wv < 4) {  // g^T v_j for this quarter, K = p
            const float* Ax = S.v + i32 * kSX + hf;
            const float* Bg = S.g + hf * kSX + 32 * tq + i32;
#pragma unroll 16
            for (int p0 = 0; p0 < kFP; p0 += 2) acc = bwd_mfma(Ax[p0], Bg[p0 * kSX], acc);
        } else if (wv == 4) {  // C.B over the half
            const float* Ac = S.C + i32 * kSX + hf;
            const float* Bbp = S.B + i32 * kSX + hf;
#pragma unroll 16
            for (int k0 = 0; k0 < 64; k0 += 2) acc = bwd_mfma(Ac[k0], Bbp[k0], acc);
        } else if (wv == 5) {  // dy.v
            const float* Ay = S.dy + i32 * kSX + hf;
            const float* Bv = S.v + i32 * kSX + hf;
#pragma unroll 16
            for (int k0 = 0; k0 < 64; k0 += 2) acc = bwd_mfma(Ay[k0], Bv[k0], acc);
        } else {  // h_c^T dy_j for this quarter, h_c from registers
            const float* Ay = S.dy + i32 * kSX + hf;
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                acc = bwd_mfma(Ay[2 * m], hreg[m], acc);
                if ((m & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
        }
        // ---- per-wave reductions
        {
            float w[16];
            if (wv < 2) {  // v_j . g B_j over this half of p
#pragma unroll
                for (int r = 0; r < 16; ++r) w[r] = acc[r] * S.v[bwd_row(r, hf) * kSX + 32 * wv + i32];
                const float s = bwd_half_sum16(w, i32);
                if ((i32 & 1) == 0) S.xu[wv][bwd_row(i32 >> 1, hf)] = s;
            } else if (wv >= 6) {  // C_k . h_c^T dy_k over this quarter; <g, h_c>
#pragma unroll
                for (int r = 0; r < 16; ++r) w[r] = acc[r] * S.C[bwd_row(r, hf) * kSX + 32 * tq + i32];
                const float s = bwd_half_sum16(w, i32);
                if ((i32 & 1) == 0) S.qh[tq][bwd_row(i32 >> 1, hf)] = s;
                float gh = 0.f;
#pragma unroll
                for (int m = 0; m < 32; ++m) gh += hreg[m] * S.g[(2 * m + hf) * kSX + 32 * tq + i32];
                gh = wave_sum(gh);
                if (lane == 0) S.ghc[tq] = gh;
                fetch_h(cn, hreg);
            } else if (wv >= 4) {
                float* dst = wv == 4 ? S.E1 : S.DX;
#pragma unroll
                for (int r = 0; r < 16; ++r) dst[bwd_row(r, hf) * kSQ + i32] = acc[r];
            }
        }
        __syncthreads();
        // ---- weighted fused Q x Q matrices: wave w takes rows 4 w .. 4 w + 3
        {
            const int i = i32, k0 = 4 * wv + 2 * hf, ti = i >> lg;
            const float cs_i = S.cs[i], sc_i = S.sc[i];
            float rs[4], xgc = 0.f;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int k = k0 + q, tk = k >> lg;
                const bool lower = tk > ti, same = tk == ti;
                const float e = lower ? __expf(S.cs[k] - cs_i) : 0.f;
                const float W = lower ? e * sc_i : (same ? S.gm[k] : 0.f);
                const float cb = S.E1[k * kSQ + i];
                const float dx = S.DX[k * kSQ + i];
                S.E1[k * kSQ + i] = W * cb;
                S.E2[k * kSQ + i] = W * dx;
                S.E3T[i * kSQ + k] = W * dx;
                rs[q] = lower ? W * dx * cb : 0.f;
                rs[2 + q] = same ? cb * dx : 0.f;
                xgc += e * cb * dx;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) rs[q] = bwd_half_sum(rs[q]);
            if (i32 < 2) {
                S.rrow[k0 + i32] = rs[i32];
                S.rdg[k0 + i32] = rs[2 + i32];
            }
            xgc += __shfl_xor(xgc, 32, 64);
            if (hf == 0) S.cpart[wv][i] = xgc;
        }
        __syncthreads();
        // ---- phase 2
        if (wv < 2) {  // dv (this half's share), p rows 32 wv ..
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] *= S.sc[bwd_row(r, hf)] * S.av[bwd_row(r, hf)];
            const float* Ap = S.E1 + hf * kSQ + i32;
            const float* Bp = S.dy + hf * kSX + 32 * wv + i32;
#pragma unroll
            for (int k0 = 0; k0 < 32; k0 += 2) acc = bwd_mfma(Ap[k0 * kSQ], Bp[k0 * kSX], acc);
            float* dvp = p.dvp + (int64_t)ns * nbl * p.M * p.H * kFP;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = bwd_row(r, hf), t = t0 + (j >> lg);
                if (t < p.L)
                    dvp[((((int64_t)b * p.L + t) * p.M + (j & (p.M - 1))) * p.H + h) * kFP + 32 * wv + i32] = acc[r];
            }
        } else if (wv < 4 || wv >= 6) {  // dB (waves 2, 3) or dC (waves 6, 7) for this quarter
            const bool isB = wv < 4;
            const float* Ap = (isB ? S.E2 : S.E3T) + hf * kSQ + i32;
            const float* Bp = (isB ? S.C : S.B) + hf * kSX + 32 * tq + i32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = bwd_row(r, hf);
                acc[r] *= isB ? S.sc[j] * S.av[j] : S.bv[j];
            }
#pragma unroll
            for (int k0 = 0; k0 < 32; k0 += 2) acc = bwd_mfma(Ap[k0 * kSQ], Bp[k0 * kSX], acc);
            float* dst = isB ? p.dBh : p.dCh;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = bwd_row(r, hf), t = t0 + (j >> lg);
                if (t < p.L)
                    dst[((((int64_t)b * p.L + t) * p.M + (j & (p.M - 1))) * p.H + h) * kFN + 64 * ns + 32 * tq + i32] =
                        acc[r];
            }
        } else {  // waves 4, 5: two tiles each of this half's g: exp(cs_end) g + sum_k b_k dy_k C_k^T
            const float dec = __expf(S.cs[31]);
            const int tp = wv - 4;
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                float* gp = S.g + (32 * tp) * kSX + 32 * tn + i32;
                bwd_f32x16 a;
#pragma unroll
                for (int r = 0; r < 16; ++r) a[r] = dec * gp[bwd_row(r, hf) * kSX];
                const float* Ap = S.dy + hf * kSX + 32 * tp + i32;
                const float* Bp = S.C + hf * kSX + 32 * tn + i32;
#pragma unroll
                for (int k0 = 0; k0 < 32; k0 += 2) a = bwd_mfma(S.bv[k0 + hf] * Ap[k0 * kSX], Bp[k0 * kSX], a);
#pragma unroll
                for (int r = 0; r < 16; ++r) gp[bwd_row(r, hf) * kSX] = a[r];
            }
        }
        if (wv == 3) {
            // per step t (lanes 0 .. QS-1): this half's share of dda, dscale, dgamma
            const int t = lane;
            const bool live = t < QS;
            const int r0 = live ? t << lg : 0;
            float xu = 0.f, qh = 0.f, xg2 = 0.f, rowm = 0.f, dg = 0.f;
            for (int m = 0; m < p.M; ++m) {
                const int j = r0 + m;
                xu += S.xu[0][j] + S.xu[1][j];
                qh += S.qh[0][j] + S.qh[1][j];
#pragma unroll
                for (int w = 0; w < 8; ++w) xg2 += S.cpart[w][j];
                rowm += S.rrow[j];
                dg += S.rdg[j];
            }
            if (!live) xu = qh = xg2 = rowm = dg = 0.f;
            const float cst = S.cs[r0], avt = S.av[r0], bvt = S.bv[r0], sct = live ? S.sc[r0] : 0.f;
            const float ghc = S.ghc[0] + S.ghc[1];
            const float scxu = sct * xu;
            float s1 = 0.f, s2 = 0.f;
            for (int u = 0; u < QS; ++u) {  // u is wave-uniform: the other step's values by lane read
                const float cu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cst), u));
                const float xuu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scxu), u));
                const float qhu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qh), u));
                if (u < t) s1 += __expf(cst - cu) * xuu;
                if (u >= t) s2 += __expf(cu - cst) * qhu;
            }
            const float colm = sct * xg2;
            const float pc = wave_incl_scan(colm) - colm;
            const float pr = wave_incl_scan(rowm) - rowm;
            if (live && t0 + t < p.L) {
                const int64_t o = (int64_t)b * p.L * p.H + (int64_t)(t0 + t) * p.H + h;
                const int64_t plane = nbl * p.H;
                p.sp[(0 * 2 + ns) * plane + o] = avt * bvt * ghc + avt * s1 + bvt * s2 + (pc - pr);
                p.sp[(1 * 2 + ns) * plane + o] = avt * xu + xg2;
                p.sp[(2 * 2 + ns) * plane + o] = dg;
            }
        }
        __syncthreads();
        b3h_commit(S, pre, tid, lg);
        __syncthreads();
    }
    for (int e = tid; e < kFP * 64; e += 512)
        p.dh0[bh * (kFP * kFN) + (e >> 6) * kFN + 64 * ns + (e & 63)] = S.g[(e >> 6) * kSX + (e & 63)];
}

// Sums of the half-dstate kernel's two partial planes (half 0 + half 1).
__global__ __launch_bounds__(256) void ssd3_bwd_half_finish(Ssd3BwdParams p) {
    const int64_t nv = (int64_t)p.nb * p.L * p.M * p.H * kFP, ns = (int64_t)p.nb * p.L * p.H;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < nv; e += stride) p.dv[e] = p.dvp[e] + p.dvp[nv + e];
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < ns; e += stride) {
        p.dda[e] = p.sp[e] + p.sp[ns + e];
        if (p.dscl) p.dscl[e] = p.sp[2 * ns + e] + p.sp[3 * ns + e];
        if (p.dgam) p.dgam[e] = p.sp[4 * ns + e] + p.sp[5 * ns + e];
    }
}

// Chunk-entry states on MFMA (headdim 64 x dstate 128), as the Mamba-2 one:
// two workgroups per (batch, head), one per 64-column half of the state; wave
// w keeps one 32 x 32 state tile as an accumulator across chunks, stores it as
// chunk c's entry state, then adds
//   exp(cs_end) h + sum_j exp(cs_end - cs_t(j)) scale_t(j) v_j B_j^T.
struct B3StatesLds {
    float v[32 * kSX];
    float B[32 * kSB];
    float w[32];
    float dec;
};

__global__ __launch_bounds__(256, 3) void ssd3_bwd_states_mfma(Ssd3BwdParams p) {
    __shared__ B3StatesLds S;
    const int tid = threadIdx.x, wv = wave_id(), lane = tid & 63, i32 = lane & 31, hf = lane >> 5;
    const int ns = blockIdx.x & 1;  // 64-column half of the state
    const int b = (blockIdx.x >> 1) / p.H, h = (blockIdx.x >> 1) % p.H, grp = h / (p.H / p.G);
    const int lg = b3_lg(p.M), mk = p.M - 1;
    const int64_t bh = (int64_t)b * p.H + h;
    const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)grp * p.B_sg;
    const int tp = wv >> 1, tn = 2 * ns + (wv & 1);
    bwd_f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        acc[r] = p.h0 ? p.h0[bh * (kFP * kFN) + (32 * tp + bwd_row(r, hf)) * kFN + 32 * tn + i32] : 0.f;
    // loads of one chunk: v rows (tid >> 4) and + 16; B rows (tid >> 5) + 8 q
    const int ix = tid >> 4, cx = (tid & 15) * 4, ib = tid >> 4, cb = 64 * ns + (tid & 15) * 4;
    float4 fv[2], fb[2];
    float fda, fsc;
    auto fetch = [&](int c) {
        const int t0 = c * p.QS;
        const float4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int j = ix + 16 * q, t = t0 + (j >> lg);
            const float4 v = *reinterpret_cast<const float4*>(vb + (int64_t)min(t, p.L - 1) * p.v_sl +
                                                              (int64_t)(j & mk) * p.v_sm + cx);
            fv[q] = t < p.L ? v : z;
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int j = ib + 16 * q, t = t0 + (j >> lg);
            const float4 v = *reinterpret_cast<const float4*>(Bb + (int64_t)min(t, p.L - 1) * p.B_sl +
                                                              (int64_t)(j & mk) * p.B_sm + cb);
            fb[q] = t < p.L ? v : z;
        }
        const int t = t0 + ((tid & 31) >> lg);
        const int64_t ot = (int64_t)min(t, p.L - 1);
        const float da = p.da[(int64_t)b * p.da_sb + ot * p.da_sl + (int64_t)h * p.da_sh];
        const float sc = p.scl ? p.scl[(int64_t)b * p.scl_sb + ot * p.scl_sl + (int64_t)h * p.scl_sh] : 1.f;
        fda = t < p.L ? da : 0.f;
        fsc = t < p.L ? sc : 0.f;
    };
    auto commit = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) bwd_put4(&S.v[(ix + 16 * q) * kSX + cx], fv[q]);
#pragma unroll
        for (int q = 0; q < 2; ++q) bwd_put4(&S.B[(ib + 16 * q) * kSB + cb], fb[q]);
        if (wv == 0) {
            const bool first = (lane & mk) == 0;
            const float cs = wave_incl_scan(lane < 32 && first ? fda : 0.f);
            const float tot = __shfl(cs, 31, 64);
            if (lane < 32) S.w[lane] = __expf(tot - cs) * fsc;
            if (lane == 31) S.dec = __expf(tot);
        }
    };
    fetch(0);
    commit();
    __syncthreads();
    for (int c = 0; c < p.nch; ++c) {
        fetch(c + 1 < p.nch ? c + 1 : c);
        float* dst = p.hs + (bh * p.nch + c) * (kFP * kFN) + (32 * tp) * kFN + i32;
        const float dec = S.dec;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dst[bwd_row(r, hf) * kFN + 32 * tn] = acc[r];
            acc[r] *= dec;
        }
        const float* Ap = S.v + hf * kSX + 32 * tp + i32;
        const float* Bp = S.B + hf * kSB + 32 * tn + i32;
#pragma unroll
        for (int k0 = 0; k0 < 32; k0 += 2) {
            const float a = S.w[k0 + hf] * Ap[k0 * kSX];
            acc = bwd_mfma(a, Bp[k0 * kSB], acc);
        }
        __syncthreads();
        commit();
        __syncthreads();
    }
}

static size_t b3_states_lds(int P, int N) { return ((size_t)P * N + (size_t)kB3F * (P + N)) * sizeof(float); }
static size_t b3_chunks_lds(int P, int N) {
    return ((size_t)2 * P * N + (size_t)3 * kB3F * P + (size_t)2 * kB3F * N + (size_t)3 * kB3F * kB3F) * sizeof(float);
}

// The MFMA path: headdim 64, dstate 128, and float4-aligned rows of v, dy, B, C.
static bool b3_mfma_ok(const mamba_ssd3_bwd_args* a) {
    auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    auto m4 = [](int64_t s0, int64_t s1, int64_t s2, int64_t s3) {
        return s0 % 4 == 0 && s1 % 4 == 0 && s2 % 4 == 0 && s3 % 4 == 0;
    };
    return a->headdim == kFP && a->dstate == kFN && al(a->v) && al(a->dy) && al(a->B) && al(a->C) &&
           m4(a->v_sb, a->v_sl, a->v_sm, a->v_sh) && m4(a->dy_sb, a->dy_sl, a->dy_sm, a->dy_sh) &&
           m4(a->B_sb, a->B_sl, a->B_sm, a->B_sg) && m4(a->C_sb, a->C_sl, a->C_sm, a->C_sg);
}

struct B3Layout {
    size_t hs, dbh, part, total;
};

static int b3_validate(const mamba_ssd3_bwd_args* a, B3Layout* lay) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->mimo > 0 && a->nheads > 0 && a->headdim > 0 &&
                        a->ngroups > 0 && a->dstate > 0,
                    "sizes must be >= 1");
    MAMBA_CHECK_ARG(kB3F % a->mimo == 0, "mimo must divide 32");
    MAMBA_CHECK_ARG(a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    MAMBA_CHECK_ARG((int64_t)a->headdim * a->dstate <= 8192, "headdim * dstate must be <= 8192");
    MAMBA_CHECK_ARG(b3_chunks_lds(a->headdim, a->dstate) <= 160 * 1024, "headdim / dstate too large for LDS");
    MAMBA_CHECK_ARG(a->v && a->da && a->B && a->C && a->dy && a->dv && a->dda && a->dB && a->dC && a->d_initial_state,
                    "v, da, B, C, dy, dv, dda, dB, dC and d_initial_state are required");
    MAMBA_CHECK_ARG(!a->dgamma || a->gamma, "dgamma needs gamma");
    MAMBA_CHECK_ARG(!a->dscale || a->scale, "dscale needs scale");
    const int64_t qs = kB3F / a->mimo;
    const int64_t nch = (a->seqlen + qs - 1) / qs;
    const int64_t bh = (int64_t)a->batch * a->nheads;
    MAMBA_CHECK_ARG(bh < (1ll << 31), "too many (batch, head) pairs");
    lay->hs = 0;
    size_t off = align_up((size_t)bh * nch * a->headdim * a->dstate * sizeof(float), 256);
    lay->dbh = off;
    if (a->ngroups != a->nheads)
        off += 2 * align_up((size_t)a->batch * a->seqlen * a->mimo * a->nheads * a->dstate * sizeof(float), 256);
    lay->part = off;
    if (b3_mfma_ok(a))  // the half-dstate kernel's partial planes
        off += align_up(2 * (size_t)a->batch * a->seqlen * a->mimo * a->nheads * a->headdim * sizeof(float), 256) +
               align_up(6 * (size_t)a->batch * a->seqlen * a->nheads * sizeof(float), 256);
    lay->total = off;
    return MAMBA_OK;
}

static int ssd3_bwd_run(const mamba_ssd3_bwd_args* a, void* workspace, size_t workspace_bytes, mamba_stream_t stream,
                        hipEvent_t ev0, hipEvent_t ev1) {
    B3Layout lay;
    const int st = b3_validate(a, &lay);
    if (st != MAMBA_OK) return st;
    if (workspace == nullptr || workspace_bytes < lay.total || ((uintptr_t)workspace & 255u) != 0) {
        set_error("mamba_ssd3_bwd: a 256-byte aligned workspace of mamba_ssd3_bwd_workspace_size() bytes is required");
        return MAMBA_ERR_WORKSPACE;
    }
    Ssd3BwdParams p;
    p.nb = a->batch; p.L = a->seqlen; p.M = a->mimo; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups;
    p.N = a->dstate; p.QS = kB3F / a->mimo; p.nch = (a->seqlen + p.QS - 1) / p.QS;
    p.v = a->v; p.v_sb = a->v_sb; p.v_sl = a->v_sl; p.v_sm = a->v_sm; p.v_sh = a->v_sh;
    p.da = a->da; p.da_sb = a->da_sb; p.da_sl = a->da_sl; p.da_sh = a->da_sh;
    p.gam = a->gamma; p.gam_sb = a->gamma_sb; p.gam_sl = a->gamma_sl; p.gam_sh = a->gamma_sh;
    p.scl = a->scale; p.scl_sb = a->scale_sb; p.scl_sl = a->scale_sl; p.scl_sh = a->scale_sh;
    p.B = a->B; p.B_sb = a->B_sb; p.B_sl = a->B_sl; p.B_sm = a->B_sm; p.B_sg = a->B_sg;
    p.C = a->C; p.C_sb = a->C_sb; p.C_sl = a->C_sl; p.C_sm = a->C_sm; p.C_sg = a->C_sg;
    p.h0 = a->initial_state;
    p.dy = a->dy; p.dy_sb = a->dy_sb; p.dy_sl = a->dy_sl; p.dy_sm = a->dy_sm; p.dy_sh = a->dy_sh;
    p.dfin = a->d_final_state;
    p.dv = a->dv; p.dda = a->dda; p.dgam = a->dgamma; p.dscl = a->dscale; p.dh0 = a->d_initial_state;
    char* ws = static_cast<char*>(workspace);
    p.hs = reinterpret_cast<float*>(ws + lay.hs);
    p.dvp = nullptr;
    p.sp = nullptr;
    if (a->ngroups == a->nheads) {
        p.dBh = a->dB;
        p.dCh = a->dC;
    } else {
        p.dBh = reinterpret_cast<float*>(ws + lay.dbh);
        p.dCh = p.dBh + align_up((size_t)a->batch * a->seqlen * a->mimo * a->nheads * a->dstate * sizeof(float), 256) /
                            sizeof(float);
    }
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(a->batch * a->nheads);
    if (b3_mfma_ok(a)) {
        p.dvp = reinterpret_cast<float*>(ws + lay.part);
        p.sp = p.dvp + align_up(2 * (size_t)a->batch * a->seqlen * a->mimo * a->nheads * a->headdim * sizeof(float), 256) /
                           sizeof(float);
        hipLaunchKernelGGL(ssd3_bwd_states_mfma, dim3(2 * grid.x), dim3(256), 0, s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
        int dev = 0, cus = 256;
        MAMBA_CHECK_HIP(hipGetDevice(&dev));
        MAMBA_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (2 * (int64_t)grid.x >= 2 * (int64_t)cus)
            hipLaunchKernelGGL(ssd3_bwd_chunks_half<4>, dim3(2 * grid.x), dim3(512), 0, s, p);
        else
            hipLaunchKernelGGL(ssd3_bwd_chunks_half<1>, dim3(2 * grid.x), dim3(512), 0, s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
        const int64_t nv = (int64_t)a->batch * a->seqlen * a->mimo * a->nheads * a->headdim;
        hipLaunchKernelGGL(ssd3_bwd_half_finish, dim3((int)std::min<int64_t>((nv + 255) / 256, 8192)), dim3(256), 0, s, p);
        MAMBA_CHECK_LAUNCH();
    } else {
        MAMBA_CHECK_HIP(hipFuncSetAttribute((const void*)ssd3_bwd_states, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)b3_states_lds(p.P, p.N)));
        MAMBA_CHECK_HIP(hipFuncSetAttribute((const void*)ssd3_bwd_chunks, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)b3_chunks_lds(p.P, p.N)));
        hipLaunchKernelGGL(ssd3_bwd_states, grid, dim3(kB3T), b3_states_lds(p.P, p.N), s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
        hipLaunchKernelGGL(ssd3_bwd_chunks, grid, dim3(kB3T), b3_chunks_lds(p.P, p.N), s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
    }
    if (a->ngroups != a->nheads) {
        const int64_t fin = (int64_t)a->batch * a->seqlen * a->mimo * a->ngroups * a->dstate;
        const int fgrid = (int)std::max<int64_t>(1, std::min<int64_t>((fin + 255) / 256, 4096));
        hipLaunchKernelGGL(ssd3_bwd_finish, dim3(fgrid), dim3(256), 0, s, p, a->dB, a->dC);
        MAMBA_CHECK_LAUNCH();
    }
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" size_t mamba_ssd3_bwd_workspace_size(const mamba_ssd3_bwd_args* a) {
    B3Layout lay;
    if (b3_validate(a, &lay) != MAMBA_OK) return 0;
    return lay.total;
}

extern "C" int mamba_ssd3_bwd(const mamba_ssd3_bwd_args* a, void* workspace, size_t workspace_bytes,
                              mamba_stream_t stream) {
    return ssd3_bwd_run(a, workspace, workspace_bytes, stream, nullptr, nullptr);
}

extern "C" int mamba_ssd3_bwd_timed(const mamba_ssd3_bwd_args* a, void* workspace, size_t workspace_bytes,
                                    mamba_stream_t stream, void* event_start, void* event_stop) {
    return ssd3_bwd_run(a, workspace, workspace_bytes, stream, (hipEvent_t)event_start, (hipEvent_t)event_stop);
}
