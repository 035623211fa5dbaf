// Mamba-2 SSD backward (recompute form), gfx950: gradients of the forward of
// ssd2.hip / ssd2_mfma.hip with respect to x, dt, A, B, C, D and the initial
// state, from dy and d(final state).
//
// Reference: the Autodiff arm of Mamba2BackendExt::ssd_serial_recalculated
// (src/mamba2/ssd/serial_recalculated/backward.rs:29-321), whose gradient math
// is src/mamba2/ssd/serial_recalculated/combined_backward.rs:126-593: the
// forward intermediates are recomputed from the saved inputs, then a reverse
// chunk loop carries the state gradient.
//
// Per (batch, head), chunks of Q = 32 positions.  With cs the within-chunk
// cumulative sum of da = dt A, e_ki = exp(cs_k - cs_i) (k >= i), a_j =
// exp(cs_end - cs_j), b_j = exp(cs_j), h_c the state entering the chunk and g
// the gradient of the state leaving it, the state after position j is
//   H_j = b_j h_c + sum_{i<=j} e_ji dt_i x_i B_i^T
// and its total gradient is
//   G_j = a_j g + sum_{k>=j} e_kj dy_k C_k^T,
// so that, without forming any P x N matrix per position:
//   dx_j = D dy_j + dt_j G_j B_j          G_j B_j = a_j g B_j + sum_k e_kj (C_k.B_j) dy_k
//   dB_j = dt_j G_j^T x_j                 G_j^T x_j = a_j g^T x_j + sum_k e_kj (dy_k.x_j) C_k
//   dC_j = H_j^T dy_j                     = b_j h_c^T dy_j + sum_{i<=j} e_ji dt_i (dy_j.x_i) B_i
//   d(da_j) = <G_j, H_j> - dt_j x_j^T G_j B_j,   ddt_j = A d(da_j) + x_j^T G_j B_j
//   <G_j, H_j> = a_j b_j <g, h_c> + a_j sum_{i<=j} e_ji dt_i x_i^T g B_i
//              + b_j sum_{k>=j} e_kj dy_k^T h_c C_k + sum_{i<=j<=k} M_ki,
//   M_ki = e_ki dt_i (dy_k.x_i)(C_k.B_i), the last sum by prefix sums of M's
//   column and row sums; dA = sum dt_j d(da_j), dD = sum x_j.dy_j, and the
//   gradient entering the previous chunk exp(cs_end) g + sum_k b_k dy_k C_k^T.
// The chunk-entry states come from a first kernel (the forward's K3 + K4),
// stored in a caller workspace.  f32 throughout; the state and its gradient
// live in LDS, so any headdim x dstate up to 64 x 128 runs.
#include <algorithm>

#include "bwd_core.h"
#include "common.h"

namespace mamba {

constexpr int kBwdQ = 32;      // positions per backward chunk
constexpr int kBwdT = 256;     // threads per workgroup

struct Ssd2BwdParams {
    int nb, L, H, P, G, N, nch;
    const float* x; int64_t x_sb, x_sl, x_sh;
    const float* dt; int64_t dt_sb, dt_sl, dt_sh;
    const float* A;
    const float* B; int64_t B_sb, B_sl, B_sg;
    const float* C; int64_t C_sb, C_sl, C_sg;
    const float* D;
    const float* h0;
    const float* dy; int64_t dy_sb, dy_sl, dy_sh;
    const float* dfin;
    float* dx; float* ddt;
    float* dBh; float* dCh;        // [b, l, h, n] per head
    float* dh0;
    float* hs;                     // [b, h, nch, P, N] chunk-entry states
    float* pA; float* pD;          // [b, h] partial sums
};

// Chunk rows into LDS: x-like [Q][P] from a [b, l, h, p] tensor, B-like [Q][N]
// from a [b, l, g, n] tensor; rows past the sequence end are zero.
__device__ __forceinline__ void bwd_rows(float* dst, const float* src, int64_t s_l, int t0, int L, int W) {
    for (int e = threadIdx.x; e < kBwdQ * W; e += kBwdT) {
        const int i = e / W, w = e - i * W;
        dst[e] = t0 + i < L ? src[(int64_t)(t0 + i) * s_l + w] : 0.f;
    }
}

// within-chunk cumulative sum of dt A (thread 0; Q = 32 terms) and its factors
__device__ __forceinline__ void bwd_cumsum(const float* dts, float A, float* cs, float* av, float* bv) {
    if (threadIdx.x == 0) {
        float run = 0.f;
        for (int i = 0; i < kBwdQ; ++i) {
            run += dts[i] * A;
            cs[i] = run;
        }
        for (int i = 0; i < kBwdQ; ++i) {
            av[i] = __expf(run - cs[i]);
            bv[i] = __expf(cs[i]);
        }
    }
}

// Chunk-entry states h_c of every chunk (the forward's K3 + K4).  One
// workgroup per (batch, head).  Dynamic LDS: [P N] state + [Q][P] x + [Q][N] B.
__global__ __launch_bounds__(kBwdT) void ssd2_bwd_states(Ssd2BwdParams p) {
    extern __shared__ float s_dyn[];
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H, g = h / (p.H / p.G);
    const int P = p.P, N = p.N, PN = P * N;
    float* hst = s_dyn;
    float* xs = hst + PN;
    float* Bs = xs + kBwdQ * P;
    __shared__ float dts[kBwdQ], cs[kBwdQ], av[kBwdQ], bv[kBwdQ];
    const int64_t bh = (int64_t)b * p.H + h;
    for (int e = threadIdx.x; e < PN; e += kBwdT) hst[e] = p.h0 ? p.h0[bh * PN + e] : 0.f;
    const float A = p.A[h];
    const float* xb = p.x + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    const float* db = p.dt + (int64_t)b * p.dt_sb + (int64_t)h * p.dt_sh;
    __syncthreads();
    for (int c = 0; c < p.nch; ++c) {
        const int t0 = c * kBwdQ;
        float* dst = p.hs + (bh * p.nch + c) * PN;
        for (int e = threadIdx.x; e < PN; e += kBwdT) dst[e] = hst[e];
        bwd_rows(xs, xb, p.x_sl, t0, p.L, P);
        bwd_rows(Bs, Bb, p.B_sl, t0, p.L, N);
        if (threadIdx.x < kBwdQ) dts[threadIdx.x] = t0 + threadIdx.x < p.L ? db[(int64_t)(t0 + threadIdx.x) * p.dt_sl] : 0.f;
        __syncthreads();
        bwd_cumsum(dts, A, cs, av, bv);
        __syncthreads();
        const float dec = __expf(cs[kBwdQ - 1]);
        for (int e = threadIdx.x; e < PN; e += kBwdT) {
            const int pp = e / N, n = e - pp * N;
            float acc = dec * hst[e];
            for (int i = 0; i < kBwdQ; ++i) acc += (av[i] * dts[i]) * xs[i * P + pp] * Bs[i * N + n];
            hst[e] = acc;
        }
        __syncthreads();
    }
}

// Block sum of one value per thread (256 threads), result in every thread.
__device__ __forceinline__ float bwd_block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// The reverse chunk loop.  One workgroup per (batch, head).  Dynamic LDS:
// g, h_c [P N]; x, dy, u/GB [Q][P]; B, C [Q][N]; e, CB, DX [Q][Q].
__global__ __launch_bounds__(kBwdT) void ssd2_bwd_chunks(Ssd2BwdParams p) {
    extern __shared__ float s_dyn[];
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H, g = h / (p.H / p.G);
    const int P = p.P, N = p.N, PN = P * N;
    constexpr int Q = kBwdQ;
    float* gs = s_dyn;              // [P][N] gradient of the state leaving the chunk
    float* hc = gs + PN;            // [P][N] state entering the chunk
    float* xs = hc + PN;            // [Q][P]
    float* dys = xs + Q * P;        // [Q][P]
    float* us = dys + Q * P;        // [Q][P]: g B_j, then G_j B_j
    float* Bs = us + Q * P;         // [Q][N]
    float* Cs = Bs + Q * N;         // [Q][N]
    float* Es = Cs + Q * N;         // [Q][Q] e_ki (k >= i)
    float* CBs = Es + Q * Q;        // [Q][Q] C_k . B_i
    float* DXs = CBs + Q * Q;       // [Q][Q] dy_k . x_i
    __shared__ float dts[Q], cs[Q], av[Q], bv[Q], xu[Q], dv[Q], colm[Q], rowm[Q], red[4];
    const int64_t bh = (int64_t)b * p.H + h;
    const float A = p.A[h], Dh = p.D ? p.D[h] : 0.f;
    const float* xb = p.x + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
    const float* yb = p.dy + (int64_t)b * p.dy_sb + (int64_t)h * p.dy_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    const float* Cb = p.C + (int64_t)b * p.C_sb + (int64_t)g * p.C_sg;
    const float* db = p.dt + (int64_t)b * p.dt_sb + (int64_t)h * p.dt_sh;
    const int tid = threadIdx.x;
    for (int e = tid; e < PN; e += kBwdT) gs[e] = p.dfin ? p.dfin[bh * PN + e] : 0.f;
    float accA = 0.f, accD = 0.f;  // per-thread partials (threads j < Q)
    for (int c = p.nch - 1; c >= 0; --c) {
        const int t0 = c * Q;
        __syncthreads();  // the previous chunk's readers of the chunk buffers are done
        const float* src = p.hs + (bh * p.nch + c) * PN;
        for (int e = tid; e < PN; e += kBwdT) hc[e] = src[e];
        bwd_rows(xs, xb, p.x_sl, t0, p.L, P);
        bwd_rows(dys, yb, p.dy_sl, t0, p.L, P);
        bwd_rows(Bs, Bb, p.B_sl, t0, p.L, N);
        bwd_rows(Cs, Cb, p.C_sl, t0, p.L, N);
        if (tid < Q) dts[tid] = t0 + tid < p.L ? db[(int64_t)(t0 + tid) * p.dt_sl] : 0.f;
        __syncthreads();
        bwd_cumsum(dts, A, cs, av, bv);
        // <g, h_c>
        float ghp = 0.f;
        for (int e = tid; e < PN; e += kBwdT) ghp += gs[e] * hc[e];
        const float ghc = bwd_block_sum(ghp, red);  // (its barriers also publish cs / av / bv)
        // Q x Q products and decays; u_j = g B_j
        for (int e = tid; e < Q * Q; e += kBwdT) {
            const int k = e / Q, i = e - k * Q;
            float cb = 0.f, dx = 0.f;
            for (int n = 0; n < N; ++n) cb += Cs[k * N + n] * Bs[i * N + n];
            for (int pp = 0; pp < P; ++pp) dx += dys[k * P + pp] * xs[i * P + pp];
            CBs[e] = cb;
            DXs[e] = dx;
            Es[e] = k >= i ? __expf(cs[k] - cs[i]) : 0.f;
        }
        for (int e = tid; e < Q * P; e += kBwdT) {
            const int j = e / P, pp = e - j * P;
            float acc = 0.f;
            for (int n = 0; n < N; ++n) acc += gs[pp * N + n] * Bs[j * N + n];
            us[e] = acc;
        }
        // dv_k = dy_k^T h_c C_k: 8 threads per k, each over P / 8 rows, then a shuffle sum
        {
            const int k = tid >> 3, part = tid & 7;
            float acc = 0.f;
            for (int pp = part; pp < P; pp += 8) {
                float v = 0.f;
                for (int n = 0; n < N; ++n) v += hc[pp * N + n] * Cs[k * N + n];
                acc += dys[k * P + pp] * v;
            }
            acc += __shfl_xor(acc, 1, 64);
            acc += __shfl_xor(acc, 2, 64);
            acc += __shfl_xor(acc, 4, 64);
            if (part == 0) dv[k] = acc;
        }
        __syncthreads();
        // x_j . g B_j; the column and row sums of M
        if (tid < Q) {
            const int j = tid;
            float a = 0.f;
            for (int pp = 0; pp < P; ++pp) a += xs[j * P + pp] * us[j * P + pp];
            xu[j] = a;
            float cm = 0.f, rm = 0.f;
            for (int k = j; k < Q; ++k) cm += Es[k * Q + j] * dts[j] * DXs[k * Q + j] * CBs[k * Q + j];
            for (int i = 0; i <= j; ++i) rm += Es[j * Q + i] * dts[i] * DXs[j * Q + i] * CBs[j * Q + i];
            colm[j] = cm;
            rowm[j] = rm;
        }
        __syncthreads();
        // G_j B_j in place of g B_j
        for (int e = tid; e < Q * P; e += kBwdT) {
            const int j = e / P, pp = e - j * P;
            float acc = av[j] * us[e];
            for (int k = j; k < Q; ++k) acc += Es[k * Q + j] * CBs[k * Q + j] * dys[k * P + pp];
            us[e] = acc;
        }
        __syncthreads();
        // per position: <G_j, H_j>, d(da_j), ddt_j, the dA / dD partials; dx_j
        if (tid < Q) {
            const int j = tid, t = t0 + j;
            float s1 = 0.f, s2 = 0.f, pre_c = 0.f, pre_r = 0.f;
            for (int i = 0; i <= j; ++i) s1 += Es[j * Q + i] * dts[i] * xu[i];
            for (int k = j; k < Q; ++k) s2 += Es[k * Q + j] * dv[k];
            for (int i = 0; i <= j; ++i) pre_c += colm[i];
            for (int k = 0; k < j; ++k) pre_r += rowm[k];
            const float gh = av[j] * bv[j] * ghc + av[j] * s1 + bv[j] * s2 + (pre_c - pre_r);
            float xgb = 0.f;
            for (int pp = 0; pp < P; ++pp) xgb += xs[j * P + pp] * us[j * P + pp];
            const float dda = gh - dts[j] * xgb;
            if (t < p.L) {
                p.ddt[(int64_t)b * p.L * p.H + (int64_t)t * p.H + h] = A * dda + xgb;
                accA += dts[j] * dda;
                accD += DXs[j * Q + j];
            }
        }
        for (int e = tid; e < Q * P; e += kBwdT) {
            const int j = e / P, pp = e - j * P;
            if (t0 + j < p.L)
                p.dx[(((int64_t)b * p.L + t0 + j) * p.H + h) * P + pp] = Dh * dys[e] + dts[j] * us[e];
        }
        // dB_j = dt_j (a_j g^T x_j + sum_k e_kj DX_kj C_k); dC_j = b_j h_c^T dy_j + sum_i e_ji dt_i DX_ji B_i
        for (int e = tid; e < Q * N; e += kBwdT) {
            const int j = e / N, n = e - j * N;
            if (t0 + j >= p.L) continue;
            float gx = 0.f, hd = 0.f;
            for (int pp = 0; pp < P; ++pp) {
                gx += gs[pp * N + n] * xs[j * P + pp];
                hd += hc[pp * N + n] * dys[j * P + pp];
            }
            float sb = av[j] * gx, sc = bv[j] * hd;
            for (int k = j; k < Q; ++k) sb += Es[k * Q + j] * DXs[k * Q + j] * Cs[k * N + n];
            for (int i = 0; i <= j; ++i) sc += Es[j * Q + i] * dts[i] * DXs[j * Q + i] * Bs[i * N + n];
            const int64_t o = (((int64_t)b * p.L + t0 + j) * p.H + h) * N + n;
            p.dBh[o] = dts[j] * sb;
            p.dCh[o] = sc;
        }
        __syncthreads();  // every reader of g for this chunk is done
        // the gradient entering this chunk: exp(cs_end) g + sum_k b_k dy_k C_k^T
        const float dec = __expf(cs[Q - 1]);
        for (int e = tid; e < PN; e += kBwdT) {
            const int pp = e / N, n = e - pp * N;
            float acc = dec * gs[e];
            for (int k = 0; k < Q; ++k) acc += bv[k] * dys[k * P + pp] * Cs[k * N + n];
            gs[e] = acc;
        }
    }
    __syncthreads();
    for (int e = tid; e < PN; e += kBwdT) p.dh0[bh * PN + e] = gs[e];
    // per-(b, h) partials, summed over the Q threads in a fixed order
    const float sA = bwd_block_sum(accA, red);
    const float sD = bwd_block_sum(accD, red);
    if (tid == 0) {
        p.pA[bh] = sA;
        p.pD[bh] = sD;
    }
}

// ---------------------------------------------------------------------------
// MFMA path for headdim 64 x dstate 128 (the config-1 head shape): the same
// recurrences with every P x N x Q and Q x Q x (P | N) contraction on
// v_mfma_f32_32x32x2_f32 (helpers in bwd_core.h).
// One chunk's inputs in registers (loaded ahead, written to LDS later).
struct BwdRows {
    float4 x, dy, B0, B1, C0, C1;
    float dt;
};

struct BwdFastLds {
    float g[kFP * kSB];      // [p][n] gradient of the state leaving the chunk
    float x[32 * kSX];       // [j][p]
    float dy[32 * kSX];      // [j][p]
    float B[32 * kSB];       // [j][n]
    float C[32 * kSB];       // [j][n]
    float E1[32 * kSQ];      // [k][i] C_k . B_i, then e_ki C_k . B_i (0 above the diagonal)
    float DX[32 * kSQ];      // [k][i] dy_k . x_i
    float E2[32 * kSQ];      // [k][i] e_ki dy_k . x_i
    float E3T[32 * kSQ];     // [i][k] e_ki dt_i dy_k . x_i
    float dt[32], cs[32], av[32], bv[32];
    float xu[2][32];         // x_j . g B_j, per 32-row half of p
    float dv[4][32];         // C_k . h_c^T dy_k, per 32-column quarter of n
    float ghc[4];            // <g, h_c>, per quarter of n
    float cpart[2][8][32];   // per-wave column sums: s2, then sum_k e_kj (C_k.B_j) (dy_k.x_j)
    float rs1[32], rrow[32]; // row sums: s1_j, and the row sums of M
};

// Loads chunk c's rows of x, dy, B, C, dt for a 512-thread block (rows past
// the sequence end read as zero; their loads are clamped to the last row).
__device__ __forceinline__ void bwd_fetch(const Ssd2BwdParams& p, const float* xb, const float* yb, const float* Bb,
                                          const float* Cb, const float* db, int c, int tid, BwdRows& f) {
    const int t0 = c * 32;
    const int ix = tid >> 4, cx = (tid & 15) * 4;
    const int ib = tid >> 5, cb = (tid & 31) * 4;
    const float4 z = {0.f, 0.f, 0.f, 0.f};
    const int tx = t0 + ix, tb0 = t0 + ib, tb1 = t0 + ib + 16, tt = t0 + (tid & 31);
    const float4 vx = *reinterpret_cast<const float4*>(xb + (int64_t)min(tx, p.L - 1) * p.x_sl + cx);
    const float4 vy = *reinterpret_cast<const float4*>(yb + (int64_t)min(tx, p.L - 1) * p.dy_sl + cx);
    const float4 vb0 = *reinterpret_cast<const float4*>(Bb + (int64_t)min(tb0, p.L - 1) * p.B_sl + cb);
    const float4 vb1 = *reinterpret_cast<const float4*>(Bb + (int64_t)min(tb1, p.L - 1) * p.B_sl + cb);
    const float4 vc0 = *reinterpret_cast<const float4*>(Cb + (int64_t)min(tb0, p.L - 1) * p.C_sl + cb);
    const float4 vc1 = *reinterpret_cast<const float4*>(Cb + (int64_t)min(tb1, p.L - 1) * p.C_sl + cb);
    const float vt = db[(int64_t)min(tt, p.L - 1) * p.dt_sl];
    f.x = tx < p.L ? vx : z;
    f.dy = tx < p.L ? vy : z;
    f.B0 = tb0 < p.L ? vb0 : z;
    f.B1 = tb1 < p.L ? vb1 : z;
    f.C0 = tb0 < p.L ? vc0 : z;
    f.C1 = tb1 < p.L ? vc1 : z;
    f.dt = tt < p.L ? vt : 0.f;
}

// Writes fetched rows to LDS; wave 0 also forms cs, a = exp(cs_end - cs),
// b = exp(cs) from dt.
__device__ __forceinline__ void bwd_commit(BwdFastLds& S, const BwdRows& f, float A, int tid) {
    const int ix = tid >> 4, cx = (tid & 15) * 4;
    const int ib = tid >> 5, cb = (tid & 31) * 4;
    bwd_put4(&S.x[ix * kSX + cx], f.x);
    bwd_put4(&S.dy[ix * kSX + cx], f.dy);
    bwd_put4(&S.B[ib * kSB + cb], f.B0);
    bwd_put4(&S.B[(ib + 16) * kSB + cb], f.B1);
    bwd_put4(&S.C[ib * kSB + cb], f.C0);
    bwd_put4(&S.C[(ib + 16) * kSB + cb], f.C1);
    if (tid < 64) {
        const int lane = tid;
        const float cs = wave_incl_scan(lane < 32 ? f.dt * A : 0.f);
        const float tot = __shfl(cs, 31, 64);
        if (lane < 32) {
            S.dt[lane] = f.dt;
            S.cs[lane] = cs;
            S.av[lane] = __expf(tot - cs);
            S.bv[lane] = __expf(cs);
        }
    }
}

// The reverse chunk loop on MFMA.  One 512-thread workgroup per (batch, head),
// eight waves with fixed roles per phase:
//   phase 1  waves 0-1: u = g B_j (one 32-column half of p each, K = n)
//            waves 2-5: g^T x_j and h_c^T dy_j (one quarter of n each, K = p;
//                       h_c's columns for the wave sit in registers)
//            wave 6: C_k . B_i;  wave 7: dy_k . x_i
//   then the Q x Q decay-weighted matrices and their row / column sums on
//   every thread, and
//   phase 2  waves 0-1: G_j B_j = a_j g B_j + sum_k e_kj (C_k.B_j) dy_k -> dx
//            waves 2-5: dB_j, dC_j (continuing the phase-1 accumulators)
//            waves 0, 1, 6, 7: the update of g (two 32 x 32 tiles each)
//            wave 7: the per-position scalars (d(da_j), ddt_j, dA / dD partials).
// The next chunk's rows (and h_c columns) are loaded during the two phases.
__global__ __launch_bounds__(512, 1) void ssd2_bwd_chunks_mfma(Ssd2BwdParams p) {
    __shared__ BwdFastLds S;
    const int tid = threadIdx.x, wv = wave_id(), lane = tid & 63, i32 = lane & 31, hf = lane >> 5;
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H, grp = h / (p.H / p.G);
    const int64_t bh = (int64_t)b * p.H + h;
    const float A = p.A[h], Dh = p.D ? p.D[h] : 0.f;
    const float* xb = p.x + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
    const float* yb = p.dy + (int64_t)b * p.dy_sb + (int64_t)h * p.dy_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)grp * p.B_sg;
    const float* Cb = p.C + (int64_t)b * p.C_sb + (int64_t)grp * p.C_sg;
    const float* db = p.dt + (int64_t)b * p.dt_sb + (int64_t)h * p.dt_sh;
    const int tq = wv - 2;  // n quarter of waves 2-5
    // h_c columns of waves 2-5: hreg[m] = h_c[2 m + hf][32 tq + i32]; reloaded
    // with the next chunk's as soon as the current chunk's last use is done
    float hreg[32];
    auto fetch_h = [&](int c, float (&dst)[32]) {
        const float* src = p.hs + (bh * p.nch + c) * (kFP * kFN) + hf * kFN + 32 * tq + i32;
#pragma unroll
        for (int m = 0; m < 32; ++m) dst[m] = src[m * 2 * kFN];
    };
    for (int e = tid; e < kFP * kFN; e += 512) S.g[(e >> 7) * kSB + (e & 127)] = p.dfin ? p.dfin[bh * (kFP * kFN) + e] : 0.f;
    BwdRows pre;
    bwd_fetch(p, xb, yb, Bb, Cb, db, p.nch - 1, tid, pre);
    if (wv >= 2 && wv < 6) fetch_h(p.nch - 1, hreg);
    bwd_commit(S, pre, A, tid);
    float accA = 0.f, accD = 0.f;
    __syncthreads();
    for (int c = p.nch - 1; c >= 0; --c) {
        const int t0 = c * 32;
        const int cn = c > 0 ? c - 1 : 0;  // the next chunk (reloads chunk 0 at the end; unused)
        // per-chunk opaque copy of the thread index: the LDS addresses derived
        // from it are then formed inside the loop instead of being hoisted out
        // of it (dozens of loop-invariant addresses would not fit in registers)
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, i32 = lane & 31, hf = lane >> 5;
        bwd_fetch(p, xb, yb, Bb, Cb, db, cn, tid, pre);
        // ---- phase 1
        bwd_f32x16 acc0 = {}, acc1 = {};
        if (wv < 2) {
            const float* Ap = S.B + i32 * kSB + hf;
            const float* Bp = S.g + (32 * wv + i32) * kSB + hf;
#pragma unroll 16
            for (int n0 = 0; n0 < kFN; n0 += 2) acc0 = bwd_mfma(Ap[n0], Bp[n0], acc0);
        } else if (wv < 6) {
            const float* Ax = S.x + i32 * kSX + hf;
            const float* Ay = S.dy + i32 * kSX + hf;
            const float* Bg = S.g + hf * kSB + 32 * tq + i32;
#pragma unroll
            for (int m = 0; m < 32; ++m) {
                acc0 = bwd_mfma(Ax[2 * m], Bg[2 * m * kSB], acc0);
                acc1 = bwd_mfma(Ay[2 * m], hreg[m], acc1);
                if ((m & 7) == 7) __builtin_amdgcn_sched_barrier(0);  // bounds the operand prefetch
            }
        } else if (wv == 6) {
            const float* Ap = S.C + i32 * kSB + hf;
            const float* Bp = S.B + i32 * kSB + hf;
#pragma unroll 16
            for (int n0 = 0; n0 < kFN; n0 += 2) acc0 = bwd_mfma(Ap[n0], Bp[n0], acc0);
        } else {
            const float* Ap = S.dy + i32 * kSX + hf;
            const float* Bp = S.x + i32 * kSX + hf;
#pragma unroll 16
            for (int p0 = 0; p0 < kFP; p0 += 2) acc0 = bwd_mfma(Ap[p0], Bp[p0], acc0);
        }
        // ---- per-wave reductions of the phase-1 products
        {
            float v[16];
            if (wv < 2) {  // x_j . g B_j over this half of p
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = acc0[r] * S.x[bwd_row(r, hf) * kSX + 32 * wv + i32];
                const float s = bwd_half_sum16(v, i32);
                if ((i32 & 1) == 0) S.xu[wv][bwd_row(i32 >> 1, hf)] = s;
            } else if (wv < 6) {  // C_k . h_c^T dy_k over this quarter of n; <g, h_c>
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = acc1[r] * S.C[bwd_row(r, hf) * kSB + 32 * tq + i32];
                const float s = bwd_half_sum16(v, i32);
                if ((i32 & 1) == 0) S.dv[tq][bwd_row(i32 >> 1, hf)] = s;
                float gh = 0.f;
#pragma unroll
                for (int m = 0; m < 32; ++m) gh += hreg[m] * S.g[(2 * m + hf) * kSB + 32 * tq + i32];
                gh = wave_sum(gh);
                if (lane == 0) S.ghc[tq] = gh;
                fetch_h(cn, hreg);
            } else {
                float* dst = wv == 6 ? S.E1 : S.DX;
#pragma unroll
                for (int r = 0; r < 16; ++r) dst[bwd_row(r, hf) * kSQ + i32] = acc0[r];
            }
        }
        __syncthreads();
        // ---- the decay-weighted Q x Q matrices; row sums s1 and M, column sums s2 and xg2
        {
            const int i = i32, k0 = 4 * wv + 2 * hf;
            const float cs_i = S.cs[i], dt_i = S.dt[i];
            const float xu_i = S.xu[0][i] + S.xu[1][i];
            float rsum[4], s2c = 0.f, xgc = 0.f;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int k = k0 + q;
                const float e = k >= i ? __expf(S.cs[k] - cs_i) : 0.f;
                const float e1 = e * S.E1[k * kSQ + i];
                const float dx = S.DX[k * kSQ + i];
                S.E1[k * kSQ + i] = e1;
                S.E2[k * kSQ + i] = e * dx;
                S.E3T[i * kSQ + k] = e * dt_i * dx;
                rsum[q] = e * dt_i * xu_i;
                rsum[2 + q] = e1 * dt_i * dx;
                s2c += e * ((S.dv[0][k] + S.dv[1][k]) + (S.dv[2][k] + S.dv[3][k]));
                xgc += e1 * dx;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) rsum[q] = bwd_half_sum(rsum[q]);
            if (i32 < 2) {
                S.rs1[k0 + i32] = rsum[i32];
                S.rrow[k0 + i32] = rsum[2 + i32];
            }
            s2c += __shfl_xor(s2c, 32, 64);
            xgc += __shfl_xor(xgc, 32, 64);
            if (hf == 0) {
                S.cpart[0][wv][i] = s2c;
                S.cpart[1][wv][i] = xgc;
            }
        }
        __syncthreads();
        // ---- phase 2
        if (wv < 2) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc0[r] *= S.av[bwd_row(r, hf)];
            const float* Ap = S.E1 + hf * kSQ + i32;
            const float* Bp = S.dy + hf * kSX + 32 * wv + i32;
#pragma unroll
            for (int k0 = 0; k0 < 32; k0 += 2) acc0 = bwd_mfma(Ap[k0 * kSQ], Bp[k0 * kSX], acc0);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = bwd_row(r, hf);
                if (t0 + j < p.L)
                    p.dx[(((int64_t)b * p.L + t0 + j) * p.H + h) * kFP + 32 * wv + i32] =
                        Dh * S.dy[j * kSX + 32 * wv + i32] + S.dt[j] * acc0[r];
            }
        } else if (wv < 6) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc0[r] *= S.av[bwd_row(r, hf)];
                acc1[r] *= S.bv[bwd_row(r, hf)];
            }
            const float* A2 = S.E2 + hf * kSQ + i32;
            const float* A3 = S.E3T + hf * kSQ + i32;
            const float* Bc = S.C + hf * kSB + 32 * tq + i32;
            const float* Bbp = S.B + hf * kSB + 32 * tq + i32;
#pragma unroll
            for (int k0 = 0; k0 < 32; k0 += 2) {
                acc0 = bwd_mfma(A2[k0 * kSQ], Bc[k0 * kSB], acc0);
                acc1 = bwd_mfma(A3[k0 * kSQ], Bbp[k0 * kSB], acc1);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = bwd_row(r, hf);
                if (t0 + j < p.L) {
                    const int64_t o = (((int64_t)b * p.L + t0 + j) * p.H + h) * kFN + 32 * tq + i32;
                    p.dBh[o] = S.dt[j] * acc0[r];
                    p.dCh[o] = acc1[r];
                }
            }
        } else if (wv == 7) {
            // per position j (lanes 0-31): <G_j, H_j>, d(da_j), ddt_j
            const int j = i32;
            const bool live = lane < 32;
            float s2 = 0.f, xg2 = 0.f;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                s2 += S.cpart[0][w][j];
                xg2 += S.cpart[1][w][j];
            }
            const float dtj = S.dt[j], avj = S.av[j], bvj = S.bv[j];
            const float xu = S.xu[0][j] + S.xu[1][j];
            const float ghc = (S.ghc[0] + S.ghc[1]) + (S.ghc[2] + S.ghc[3]);
            const float colm = live ? dtj * xg2 : 0.f, rowm = live ? S.rrow[j] : 0.f;
            const float pc = wave_incl_scan(colm);
            const float pr = wave_incl_scan(rowm) - rowm;
            const float gh = avj * bvj * ghc + avj * S.rs1[j] + bvj * s2 + (pc - pr);
            const float xgb = avj * xu + xg2;
            const float dda = gh - dtj * xgb;
            if (live && t0 + j < p.L) {
                p.ddt[(int64_t)b * p.L * p.H + (int64_t)(t0 + j) * p.H + h] = A * dda + xgb;
                accA += dtj * dda;
                accD += S.DX[j * kSQ + j];
            }
        }
        // the gradient entering this chunk: exp(cs_end) g + sum_k b_k dy_k C_k^T
        if (wv < 2 || wv >= 6) {
            const float dec = __expf(S.cs[31]);
            const int gt0 = wv < 2 ? 2 * wv : 2 * wv - 8;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int tile = gt0 + tt, tp = tile >> 2, tn = tile & 3;
                float* gp = S.g + (32 * tp) * kSB + 32 * tn + i32;
                bwd_f32x16 a;
#pragma unroll
                for (int r = 0; r < 16; ++r) a[r] = dec * gp[bwd_row(r, hf) * kSB];
                const float* Ap = S.dy + hf * kSX + 32 * tp + i32;
                const float* Bp = S.C + hf * kSB + 32 * tn + i32;
#pragma unroll
                for (int k0 = 0; k0 < 32; k0 += 2) a = bwd_mfma(S.bv[k0 + hf] * Ap[k0 * kSX], Bp[k0 * kSB], a);
#pragma unroll
                for (int r = 0; r < 16; ++r) gp[bwd_row(r, hf) * kSB] = a[r];
            }
        }
        __syncthreads();
        bwd_commit(S, pre, A, tid);
        __syncthreads();
    }
    for (int e = tid; e < kFP * kFN; e += 512) p.dh0[bh * (kFP * kFN) + e] = S.g[(e >> 7) * kSB + (e & 127)];
    if (wv == 7) {
        const float sA = wave_sum(accA), sD = wave_sum(accD);
        if (lane == 0) {
            p.pA[bh] = sA;
            p.pD[bh] = sD;
        }
    }
}

// Chunk-entry states on MFMA (headdim 64 x dstate 128): two 256-thread
// workgroups per (batch, head), one per 64-column half of the state (the
// columns evolve independently); wave w keeps one 32 x 32 tile (rows
// 32 (w / 2).., columns 32 (2 half + w % 2)..) as an accumulator across
// chunks, stores it as chunk c's entry state, then adds
//   exp(cs_end) h + sum_i exp(cs_end - cs_i) dt_i x_i B_i^T.
struct BwdStatesLds {
    float x[32 * kSX];
    float B[32 * kSB];
    float w[32];
    float dec;
};

__global__ __launch_bounds__(256, 3) void ssd2_bwd_states_mfma(Ssd2BwdParams p) {
    __shared__ BwdStatesLds S;
    const int tid = threadIdx.x, wv = wave_id(), lane = tid & 63, i32 = lane & 31, hf = lane >> 5;
    const int ns = blockIdx.x & 1;  // 64-column half of the state
    const int b = (blockIdx.x >> 1) / p.H, h = (blockIdx.x >> 1) % p.H, grp = h / (p.H / p.G);
    const int64_t bh = (int64_t)b * p.H + h;
    const float A = p.A[h];
    const float* xb = p.x + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
    const float* Bb = p.B + (int64_t)b * p.B_sb + (int64_t)grp * p.B_sg;
    const float* db = p.dt + (int64_t)b * p.dt_sb + (int64_t)h * p.dt_sh;
    const int tp = wv >> 1, tn = 2 * ns + (wv & 1);
    bwd_f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        acc[r] = p.h0 ? p.h0[bh * (kFP * kFN) + (32 * tp + bwd_row(r, hf)) * kFN + 32 * tn + i32] : 0.f;
    // loads of one chunk: x rows (tid >> 4) and + 16; B rows (tid >> 5) + 8 q
    const int ix = tid >> 4, cx = (tid & 15) * 4, ib = tid >> 4, cb = 64 * ns + (tid & 15) * 4;
    float4 fx[2], fb[2];
    float fdt;
    auto fetch = [&](int c) {
        const int t0 = c * 32;
        const float4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int t = t0 + ix + 16 * q;
            const float4 v = *reinterpret_cast<const float4*>(xb + (int64_t)min(t, p.L - 1) * p.x_sl + cx);
            fx[q] = t < p.L ? v : z;
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int t = t0 + ib + 16 * q;
            const float4 v = *reinterpret_cast<const float4*>(Bb + (int64_t)min(t, p.L - 1) * p.B_sl + cb);
            fb[q] = t < p.L ? v : z;
        }
        const int t = t0 + (tid & 31);
        const float v = db[(int64_t)min(t, p.L - 1) * p.dt_sl];
        fdt = t < p.L ? v : 0.f;
    };
    auto commit = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) bwd_put4(&S.x[(ix + 16 * q) * kSX + cx], fx[q]);
#pragma unroll
        for (int q = 0; q < 2; ++q) bwd_put4(&S.B[(ib + 16 * q) * kSB + cb], fb[q]);
        if (wv == 0) {
            const float cs = wave_incl_scan(lane < 32 ? fdt * A : 0.f);
            const float tot = __shfl(cs, 31, 64);
            if (lane < 32) S.w[lane] = __expf(tot - cs) * fdt;
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
        const float* Ap = S.x + hf * kSX + 32 * tp + i32;
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

// dA[h], dD[h] = sum over the batch of the (b, h) partials; dB / dC summed over
// the heads of each group (in head order) when ngroups < nheads.
__global__ __launch_bounds__(256) void ssd2_bwd_finish(Ssd2BwdParams p, float* dA, float* dD, float* dB, float* dC) {
    const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (tid < p.H) {
        float a = 0.f, d = 0.f;
        for (int b = 0; b < p.nb; ++b) {
            a += p.pA[(int64_t)b * p.H + tid];
            d += p.pD[(int64_t)b * p.H + tid];
        }
        dA[tid] = a;
        if (dD) dD[tid] = d;
    }
    if (p.G == p.H) return;  // per-head B / C: the kernel wrote dB / dC directly
    const int rep = p.H / p.G;
    const int64_t total = (int64_t)p.nb * p.L * p.G * p.N;
    for (int64_t e = tid; e < total; e += (int64_t)gridDim.x * 256) {
        const int n = (int)(e % p.N);
        const int64_t r = e / p.N;
        const int gg = (int)(r % p.G);
        const int64_t bl = r / p.G;
        float sb = 0.f, sc = 0.f;
        for (int k = 0; k < rep; ++k) {
            const int64_t o = (bl * p.H + (int64_t)gg * rep + k) * p.N + n;
            sb += p.dBh[o];
            sc += p.dCh[o];
        }
        dB[e] = sb;
        dC[e] = sc;
    }
}

static size_t bwd_states_lds(int P, int N) { return ((size_t)P * N + (size_t)kBwdQ * (P + N)) * sizeof(float); }
static size_t bwd_chunks_lds(int P, int N) {
    return ((size_t)2 * P * N + (size_t)3 * kBwdQ * P + (size_t)2 * kBwdQ * N + (size_t)3 * kBwdQ * kBwdQ) * sizeof(float);
}

struct BwdLayout {
    size_t hs, dbh, pa, total;
};

// The MFMA path: headdim 64, dstate 128, and float4-aligned rows of x, dy, B, C.
static bool bwd_mfma_ok(const mamba_ssd2_bwd_args* a) {
    auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    auto m4 = [](int64_t s0, int64_t s1, int64_t s2) { return s0 % 4 == 0 && s1 % 4 == 0 && s2 % 4 == 0; };
    return a->headdim == kFP && a->dstate == kFN && al(a->x) && al(a->dy) && al(a->B) && al(a->C) &&
           m4(a->x_sb, a->x_sl, a->x_sh) && m4(a->dy_sb, a->dy_sl, a->dy_sh) && m4(a->B_sb, a->B_sl, a->B_sg) &&
           m4(a->C_sb, a->C_sl, a->C_sg);
}

static int bwd_validate(const mamba_ssd2_bwd_args* a, BwdLayout* lay) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->nheads > 0 && a->headdim > 0 && a->ngroups > 0 && a->dstate > 0,
                    "sizes must be >= 1");
    MAMBA_CHECK_ARG(a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    MAMBA_CHECK_ARG((int64_t)a->headdim * a->dstate <= 8192, "headdim * dstate must be <= 8192");
    MAMBA_CHECK_ARG(bwd_chunks_lds(a->headdim, a->dstate) <= 160 * 1024, "headdim / dstate too large for LDS");
    MAMBA_CHECK_ARG(a->x && a->dt && a->A && a->B && a->C && a->dy && a->dx && a->ddt && a->dA && a->dB && a->dC &&
                        a->d_initial_state,
                    "x, dt, A, B, C, dy and every gradient but dD are required");
    MAMBA_CHECK_ARG(!a->dD || a->D, "dD needs D");
    const int64_t nch = (a->seqlen + kBwdQ - 1) / kBwdQ;
    const int64_t bh = (int64_t)a->batch * a->nheads;
    MAMBA_CHECK_ARG(bh < (1ll << 31), "too many (batch, head) pairs");
    lay->hs = 0;
    size_t off = align_up((size_t)bh * nch * a->headdim * a->dstate * sizeof(float), 256);
    lay->dbh = off;
    if (a->ngroups != a->nheads) off += 2 * align_up((size_t)a->batch * a->seqlen * a->nheads * a->dstate * sizeof(float), 256);
    lay->pa = off;
    off += 2 * align_up((size_t)bh * sizeof(float), 256);
    lay->total = off;
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" size_t mamba_ssd2_bwd_workspace_size(const mamba_ssd2_bwd_args* a) {
    BwdLayout lay;
    if (bwd_validate(a, &lay) != MAMBA_OK) return 0;
    return lay.total;
}

static int ssd2_bwd_run(const mamba_ssd2_bwd_args* a, void* workspace, size_t workspace_bytes,
                        mamba_stream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    BwdLayout lay;
    const int st = bwd_validate(a, &lay);
    if (st != MAMBA_OK) return st;
    if (workspace == nullptr || workspace_bytes < lay.total || ((uintptr_t)workspace & 255u) != 0) {
        set_error("mamba_ssd2_bwd: a 256-byte aligned workspace of mamba_ssd2_bwd_workspace_size() bytes is required");
        return MAMBA_ERR_WORKSPACE;
    }
    Ssd2BwdParams p;
    p.nb = a->batch; p.L = a->seqlen; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups; p.N = a->dstate;
    p.nch = (a->seqlen + kBwdQ - 1) / kBwdQ;
    p.x = a->x; p.x_sb = a->x_sb; p.x_sl = a->x_sl; p.x_sh = a->x_sh;
    p.dt = a->dt; p.dt_sb = a->dt_sb; p.dt_sl = a->dt_sl; p.dt_sh = a->dt_sh;
    p.A = a->A;
    p.B = a->B; p.B_sb = a->B_sb; p.B_sl = a->B_sl; p.B_sg = a->B_sg;
    p.C = a->C; p.C_sb = a->C_sb; p.C_sl = a->C_sl; p.C_sg = a->C_sg;
    p.D = a->D; p.h0 = a->initial_state;
    p.dy = a->dy; p.dy_sb = a->dy_sb; p.dy_sl = a->dy_sl; p.dy_sh = a->dy_sh;
    p.dfin = a->d_final_state;
    p.dx = a->dx; p.ddt = a->ddt; p.dh0 = a->d_initial_state;
    char* ws = static_cast<char*>(workspace);
    p.hs = reinterpret_cast<float*>(ws + lay.hs);
    if (a->ngroups == a->nheads) {
        p.dBh = a->dB;
        p.dCh = a->dC;
    } else {
        p.dBh = reinterpret_cast<float*>(ws + lay.dbh);
        p.dCh = p.dBh + align_up((size_t)a->batch * a->seqlen * a->nheads * a->dstate * sizeof(float), 256) / sizeof(float);
    }
    p.pA = reinterpret_cast<float*>(ws + lay.pa);
    p.pD = p.pA + align_up((size_t)a->batch * a->nheads * sizeof(float), 256) / sizeof(float);
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(a->batch * a->nheads);
    if (bwd_mfma_ok(a)) {
        hipLaunchKernelGGL(ssd2_bwd_states_mfma, dim3(2 * grid.x), dim3(256), 0, s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
        hipLaunchKernelGGL(ssd2_bwd_chunks_mfma, grid, dim3(512), 0, s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
    } else {
        // dynamic LDS above the 64 KB default (up to the CU's 160 KB)
        MAMBA_CHECK_HIP(hipFuncSetAttribute((const void*)ssd2_bwd_states, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)bwd_states_lds(p.P, p.N)));
        MAMBA_CHECK_HIP(hipFuncSetAttribute((const void*)ssd2_bwd_chunks, hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)bwd_chunks_lds(p.P, p.N)));
        hipLaunchKernelGGL(ssd2_bwd_states, grid, dim3(kBwdT), bwd_states_lds(p.P, p.N), s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
        hipLaunchKernelGGL(ssd2_bwd_chunks, grid, dim3(kBwdT), bwd_chunks_lds(p.P, p.N), s, p);
        MAMBA_CHECK_LAUNCH();
        if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
    }
    const int64_t fin = a->ngroups == a->nheads ? 0 : (int64_t)a->batch * a->seqlen * a->ngroups * a->dstate;
    const int fgrid = (int)std::max<int64_t>((a->nheads + 255) / 256, std::min<int64_t>((fin + 255) / 256, 4096));
    hipLaunchKernelGGL(ssd2_bwd_finish, dim3(fgrid), dim3(256), 0, s, p, a->dA, a->dD, a->dB, a->dC);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

extern "C" int mamba_ssd2_bwd(const mamba_ssd2_bwd_args* a, void* workspace, size_t workspace_bytes,
                              mamba_stream_t stream) {
    return ssd2_bwd_run(a, workspace, workspace_bytes, stream, nullptr, nullptr);
}

extern "C" int mamba_ssd2_bwd_timed(const mamba_ssd2_bwd_args* a, void* workspace, size_t workspace_bytes,
                                    mamba_stream_t stream, void* event_start, void* event_stop) {
    return ssd2_bwd_run(a, workspace, workspace_bytes, stream, (hipEvent_t)event_start, (hipEvent_t)event_stop);
}
