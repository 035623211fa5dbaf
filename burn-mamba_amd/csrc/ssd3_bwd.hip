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

static size_t b3_states_lds(int P, int N) { return ((size_t)P * N + (size_t)kB3F * (P + N)) * sizeof(float); }
static size_t b3_chunks_lds(int P, int N) {
    return ((size_t)2 * P * N + (size_t)3 * kB3F * P + (size_t)2 * kB3F * N + (size_t)3 * kB3F * kB3F) * sizeof(float);
}

struct B3Layout {
    size_t hs, dbh, total;
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
