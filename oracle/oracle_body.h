/*
 * CPU restatement of swfsql/burn-mamba's SSM hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This file is the parity oracle.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker or as the
 * timed CPU baseline; the product path (burn-mamba_amd/) never links it.
 *
 * It is compiled twice by oracle.c: REAL=float (the reference's own f32 Burn
 * arithmetic, op for op) and REAL=double (a high-precision "truth").  Inputs
 * and outputs are always float; REAL is the type every intermediate is held in.
 *
 * Every function cites the reference file:line it restates.  The reference is
 * Rust over Burn (no Rust toolchain and no Burn sources exist here), so the
 * restatement is pinned by relational and closed-form checks in
 * tests/test_oracle.py rather than by running the reference.
 *
 * Memory layouts (row-major, innermost last):
 *   Mamba-2 SSD : x[b,l,h,p] dt[b,l,h] A[h] B,C[b,l,g,n] D[h] h0,hT[b,h,p,n]
 *                 y[b,l,h,p]; head h reads group h / (H/G)  (gqa.rs:30-56)
 *   Mamba-1 scan: u,delta,z,y[b,d,l] A[d,n] B,C[b,n,l] D[d] h0,hT[b,d,n]
 *   Mamba-3 SSD : v[b,l,m,h,p] da,gamma,scale[b,l,h] B,C[b,l,m,h,n]
 *                 h0,hT[b,h,p,n] y[b,l,m,h,p]
 */

#ifndef REAL
#error "define REAL and PFX before including oracle_body.h"
#endif

#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define F(name) CAT(PFX, name)

static inline REAL F(exp_)(REAL v) { return (REAL)exp((double)v); }

/* src/modules/activation/softplus.rs:17-48 — x above the per-dtype threshold
 * passes through, else log1p(exp(min(x, thr))).  Both precisions use the f32
 * model's threshold (18): prec=64 evaluates the f32 model's formula in f64
 * arithmetic, which is the truth the f32/bf16 GPU path is checked against. */
static inline REAL F(softplus_)(REAL v) {
    const REAL thr = (REAL)18;
    if (v > thr) return v;
    return (REAL)log1p(exp((double)(v < thr ? v : thr)));
}

/* src/modules/activation/silu.rs:24-27 — x / (1 + exp(-x)). */
static inline REAL F(silu_)(REAL v) { return v / ((REAL)exp(-(double)v) + (REAL)1); }

/* src/utils/mod.rs:59-65 — div_eps(F32) = 8.1584695e-8, the f32 model's
 * constant, at both precisions (see softplus_ above). */
static inline REAL F(div_eps_)(void) { return (REAL)8.1584695e-8f; }

/* ------------------------------------------------------------------------- */
/* Mamba-2 SSD, serial K1..K5 — src/mamba2/ssd/serial.rs:34-506 (identical to */
/* the trait default body serial_recalculated.rs:98-155).  The sequence is    */
/* zero-padded to a chunk multiple exactly as Mamba2::forward does            */
/* (src/mamba2/mamba2.rs:709-722): dt = 0 there, so the pad is an identity.   */
/* init_hpr (learnable initial state) is added to h0 as ssd_minimal does      */
/* (minimal.rs:316-328); the serial path itself asserts it is None.           */
/* ------------------------------------------------------------------------- */
void F(ssd2_serial)(int batch, int seqlen, int nheads, int headdim, int ngroups, int dstate,
                    int chunk, const float* x, const float* dt, const float* A, const float* B,
                    const float* C, const float* D, const float* h0, const float* init_hpr,
                    float* y, float* hT) {
    const int P = headdim, N = dstate, H = nheads, G = ngroups, Q = chunk;
    const int nch = (seqlen + Q - 1) / Q;
    const int hpg = H / G;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            const int g = h / hpg;
            REAL* cs = (REAL*)calloc((size_t)nch * Q, sizeof(REAL));
            REAL* S = (REAL*)calloc((size_t)nch * P * N, sizeof(REAL));
            REAL* hin = (REAL*)calloc((size_t)nch * P * N, sizeof(REAL));
            REAL* run = (REAL*)calloc((size_t)P * N, sizeof(REAL));
            REAL* cb = (REAL*)calloc((size_t)Q * Q, sizeof(REAL));
            REAL* wsc = (REAL*)calloc((size_t)Q, sizeof(REAL));
#define T_OF(c, l) ((c) * Q + (l))
#define DT(t) ((t) < seqlen ? (REAL)dt[((size_t)b * seqlen + (t)) * H + h] : (REAL)0)
#define XV(t, p) ((t) < seqlen ? (REAL)x[(((size_t)b * seqlen + (t)) * H + h) * P + (p)] : (REAL)0)
#define BV(t, n) ((t) < seqlen ? (REAL)B[(((size_t)b * seqlen + (t)) * G + g) * N + (n)] : (REAL)0)
#define CV(t, n) ((t) < seqlen ? (REAL)C[(((size_t)b * seqlen + (t)) * G + g) * N + (n)] : (REAL)0)
            /* K1 — serial.rs:138-164: da_cs = cumsum_l(dt * A) per chunk. */
            for (int c = 0; c < nch; ++c) {
                REAL acc = 0;
                for (int l = 0; l < Q; ++l) {
                    acc += DT(T_OF(c, l)) * (REAL)A[h];
                    cs[T_OF(c, l)] = acc;
                }
            }
            /* K3 — serial.rs:192-268: S = x^T (B * (exp(da_end - da_cs) * dt)). */
            for (int c = 0; c < nch; ++c) {
                const REAL end = cs[T_OF(c, Q - 1)];
                for (int l = 0; l < Q; ++l) wsc[l] = F(exp_)(end - cs[T_OF(c, l)]) * DT(T_OF(c, l));
                REAL* Sc = S + (size_t)c * P * N;
                for (int l = 0; l < Q; ++l) {
                    const int t = T_OF(c, l);
                    if (t >= seqlen) break;
                    for (int p = 0; p < P; ++p) {
                        const REAL xv = XV(t, p);
                        for (int n = 0; n < N; ++n) Sc[p * N + n] += xv * (BV(t, n) * wsc[l]);
                    }
                }
            }
            /* K4 — serial.rs:275-343: running = exp(da_end) * running + S. */
            for (int i = 0; i < P * N; ++i) {
                REAL v0 = h0 ? (REAL)h0[((size_t)b * H + h) * P * N + i] : (REAL)0;
                if (init_hpr) v0 += (REAL)init_hpr[(size_t)h * P * N + i];
                run[i] = v0;
            }
            for (int c = 0; c < nch; ++c) {
                const REAL dec = F(exp_)(cs[T_OF(c, Q - 1)]);
                memcpy(hin + (size_t)c * P * N, run, sizeof(REAL) * P * N);
                for (int i = 0; i < P * N; ++i) run[i] = dec * run[i] + S[(size_t)c * P * N + i];
            }
            for (int i = 0; i < P * N; ++i) hT[((size_t)b * H + h) * P * N + i] = (float)run[i];
            /* K2 + K5 — serial.rs:170-185, 349-506. */
            for (int c = 0; c < nch; ++c) {
                for (int i = 0; i < Q; ++i)
                    for (int j = 0; j < Q; ++j) {
                        REAL acc = 0;
                        for (int n = 0; n < N; ++n) acc += CV(T_OF(c, i), n) * BV(T_OF(c, j), n);
                        cb[i * Q + j] = acc;
                    }
                const REAL* hc = hin + (size_t)c * P * N;
                for (int i = 0; i < Q; ++i) {
                    const int ti = T_OF(c, i);
                    if (ti >= seqlen) break;
                    const REAL edi = F(exp_)(cs[ti]);
                    for (int p = 0; p < P; ++p) {
                        REAL blue = 0;
                        for (int n = 0; n < N; ++n) blue += CV(ti, n) * hc[p * N + n];
                        blue *= edi;
                        REAL orange = 0;
                        for (int j = 0; j <= i; ++j) {
                            const int tj = T_OF(c, j);
                            orange += ((cb[i * Q + j] * F(exp_)(cs[ti] - cs[tj])) * DT(tj)) * XV(tj, p);
                        }
                        const REAL skip = (D ? (REAL)D[h] : (REAL)0) * XV(ti, p);
                        y[(((size_t)b * seqlen + ti) * H + h) * P + p] = (float)((blue + orange) + skip);
                    }
                }
            }
#undef T_OF
#undef DT
#undef XV
#undef BV
#undef CV
            free(cs); free(S); free(hin); free(run); free(cb); free(wsc);
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-2 SSD, minimal (segsum) form — src/mamba2/ssd/minimal.rs:95-496,     */
/* segsum src/modules/misc/segsum.rs:35-47.  Different association from the  */
/* serial form (B-bar = dt*B inside C.B^T; O(nchunks^2) state passing), so    */
/* agreement with ssd2_serial pins both.                                      */
/* ------------------------------------------------------------------------- */
void F(ssd2_minimal)(int batch, int seqlen, int nheads, int headdim, int ngroups, int dstate,
                     int chunk, const float* x, const float* dt, const float* A, const float* B,
                     const float* C, const float* D, const float* h0, const float* init_hpr,
                     float* y, float* hT) {
    const int P = headdim, N = dstate, H = nheads, G = ngroups, Q = chunk;
    const int nch = (seqlen + Q - 1) / Q;
    const int hpg = H / G;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            const int g = h / hpg;
            const size_t PN = (size_t)P * N;
            REAL* cs = (REAL*)calloc((size_t)nch * Q, sizeof(REAL));
            REAL* st = (REAL*)calloc((size_t)(nch + 1) * PN, sizeof(REAL)); /* [h0, s_0..s_{n-1}] */
            REAL* ns = (REAL*)calloc((size_t)(nch + 1) * PN, sizeof(REAL));
            REAL* csN = (REAL*)calloc((size_t)(nch + 1), sizeof(REAL));
#define T_OF(c, l) ((c) * Q + (l))
#define DT(t) ((t) < seqlen ? (REAL)dt[((size_t)b * seqlen + (t)) * H + h] : (REAL)0)
#define XV(t, p) ((t) < seqlen ? (REAL)x[(((size_t)b * seqlen + (t)) * H + h) * P + (p)] : (REAL)0)
#define BV(t, n) ((t) < seqlen ? (REAL)B[(((size_t)b * seqlen + (t)) * G + g) * N + (n)] : (REAL)0)
#define CV(t, n) ((t) < seqlen ? (REAL)C[(((size_t)b * seqlen + (t)) * G + g) * N + (n)] : (REAL)0)
            /* a_cumsum (minimal.rs:121-141). */
            for (int c = 0; c < nch; ++c) {
                REAL acc = 0;
                for (int l = 0; l < Q; ++l) { acc += DT(T_OF(c, l)) * (REAL)A[h]; cs[T_OF(c, l)] = acc; }
            }
            /* STEP 2 chunk states (minimal.rs:229-286). */
            for (size_t i = 0; i < PN; ++i) {
                REAL v0 = h0 ? (REAL)h0[((size_t)b * H + h) * PN + i] : (REAL)0;
                if (init_hpr) v0 += (REAL)init_hpr[(size_t)h * PN + i];
                st[i] = v0;
            }
            for (int c = 0; c < nch; ++c) {
                REAL* s = st + (size_t)(c + 1) * PN;
                const REAL end = cs[T_OF(c, Q - 1)];
                for (int l = 0; l < Q; ++l) {
                    const int t = T_OF(c, l);
                    if (t >= seqlen) break;
                    const REAL dec = F(exp_)(end - cs[t]);
                    for (int p = 0; p < P; ++p) {
                        const REAL dx = dec * XV(t, p);
                        for (int n = 0; n < N; ++n) s[p * N + n] += dx * (DT(t) * BV(t, n));
                    }
                }
            }
            /* STEP 3 inter-chunk segsum scan (minimal.rs:288-389). */
            csN[0] = 0;
            for (int c = 0; c < nch; ++c) csN[c + 1] = csN[c] + cs[T_OF(c, Q - 1)];
            for (int i = 0; i <= nch; ++i)
                for (int j = 0; j <= i; ++j) {
                    const REAL w = F(exp_)(csN[i] - csN[j]);
                    for (size_t e = 0; e < PN; ++e) ns[(size_t)i * PN + e] += w * st[(size_t)j * PN + e];
                }
            for (size_t e = 0; e < PN; ++e) hT[((size_t)b * H + h) * PN + e] = (float)ns[(size_t)nch * PN + e];
            /* STEP 1 (Y_diag) + STEP 4 (Y_off) + D skip (minimal.rs:143-227, 391-494). */
            for (int c = 0; c < nch; ++c) {
                const REAL* hc = ns + (size_t)c * PN;
                for (int i = 0; i < Q; ++i) {
                    const int ti = T_OF(c, i);
                    if (ti >= seqlen) break;
                    for (int p = 0; p < P; ++p) {
                        REAL yd = 0;
                        for (int j = 0; j <= i; ++j) {
                            const int tj = T_OF(c, j);
                            REAL cbv = 0;
                            for (int n = 0; n < N; ++n) cbv += CV(ti, n) * (DT(tj) * BV(tj, n));
                            yd += (cbv * F(exp_)(cs[ti] - cs[tj])) * XV(tj, p);
                        }
                        REAL ch = 0;
                        for (int n = 0; n < N; ++n) ch += CV(ti, n) * hc[p * N + n];
                        const REAL yo = ch * F(exp_)(cs[ti]);
                        const REAL yv = (yd + yo) + (D ? (REAL)D[h] : (REAL)0) * XV(ti, p);
                        y[(((size_t)b * seqlen + ti) * H + h) * P + p] = (float)yv;
                    }
                }
            }
#undef T_OF
#undef DT
#undef XV
#undef BV
#undef CV
            free(cs); free(st); free(ns); free(csN);
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-2 token-by-token recurrence — the SSM update of Mamba2::step         */
/* (src/mamba2/mamba2.rs:932-991) applied to every position:                  */
/*   h = h * exp(dt*A) + (dt*B)*x ;  y = sum_n h*C + D*x                      */
/* ------------------------------------------------------------------------- */
void F(ssd2_recurrent)(int batch, int seqlen, int nheads, int headdim, int ngroups, int dstate,
                       const float* x, const float* dt, const float* A, const float* B,
                       const float* C, const float* D, const float* h0, const float* init_hpr,
                       float* y, float* hT) {
    const int P = headdim, N = dstate, H = nheads, G = ngroups;
    const int hpg = H / G;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            const int g = h / hpg;
            const size_t PN = (size_t)P * N;
            REAL* s = (REAL*)calloc(PN, sizeof(REAL));
            for (size_t i = 0; i < PN; ++i) {
                REAL v0 = h0 ? (REAL)h0[((size_t)b * H + h) * PN + i] : (REAL)0;
                if (init_hpr) v0 += (REAL)init_hpr[(size_t)h * PN + i];
                s[i] = v0;
            }
            for (int t = 0; t < seqlen; ++t) {
                const REAL dtv = dt[((size_t)b * seqlen + t) * H + h];
                const REAL dA = F(exp_)(dtv * (REAL)A[h]);
                const float* xr = x + (((size_t)b * seqlen + t) * H + h) * P;
                const float* br = B + (((size_t)b * seqlen + t) * G + g) * N;
                const float* cr = C + (((size_t)b * seqlen + t) * G + g) * N;
                for (int p = 0; p < P; ++p) {
                    REAL acc = 0;
                    for (int n = 0; n < N; ++n) {
                        s[p * N + n] = s[p * N + n] * dA + (dtv * (REAL)br[n]) * (REAL)xr[p];
                        acc += s[p * N + n] * (REAL)cr[n];
                    }
                    y[(((size_t)b * seqlen + t) * H + h) * P + p] =
                        (float)(acc + (D ? (REAL)D[h] : (REAL)0) * (REAL)xr[p]);
                }
            }
            for (size_t i = 0; i < PN; ++i) hT[((size_t)b * H + h) * PN + i] = (float)s[i];
            free(s);
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-1 selective scan — src/mamba1/mamba1.rs:422-523 (sequential loop     */
/* :496-510), plus the optional Burn softplus of delta (mamba1.rs:391-394:    */
/* dt_proj bias then softplus(., beta=1)) and the silu(z) gate applied by     */
/* Mamba1::forward (mamba1.rs:348).                                           */
/*   a = exp(delta*A) ; h = h*a + (delta*B)*u ; y = h.C ; y += D*u ; y*=silu(z)*/
/* ------------------------------------------------------------------------- */
void F(mamba1_scan)(int batch, int dim, int seqlen, int dstate, const float* u, const float* delta,
                    const float* A, const float* B, const float* C, const float* D,
                    const float* z, const float* delta_bias, int delta_softplus, const float* h0,
                    float* y, float* hT) {
    const int N = dstate, L = seqlen;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < batch; ++b)
        for (int d = 0; d < dim; ++d) {
            REAL s[256];
            for (int n = 0; n < N; ++n) s[n] = h0 ? (REAL)h0[((size_t)b * dim + d) * N + n] : (REAL)0;
            const size_t row = ((size_t)b * dim + d) * L;
            for (int t = 0; t < L; ++t) {
                REAL dl = delta[row + t];
                if (delta_bias) dl += (REAL)delta_bias[d];
                /* Burn activation::softplus(x, 1) = log(1 + exp(x)) (no threshold). */
                if (delta_softplus) dl = (REAL)log1p(exp((double)dl));
                const REAL uv = u[row + t];
                REAL acc = 0;
                for (int n = 0; n < N; ++n) {
                    const REAL a = F(exp_)(dl * (REAL)A[(size_t)d * N + n]);
                    const REAL bu = (dl * (REAL)B[((size_t)b * N + n) * L + t]) * uv;
                    s[n] = s[n] * a + bu;
                    acc += s[n] * (REAL)C[((size_t)b * N + n) * L + t];
                }
                REAL out = acc + (D ? (REAL)D[d] : (REAL)0) * uv;
                if (z) out *= F(silu_)((REAL)z[row + t]);
                y[row + t] = (float)out;
            }
            if (hT)
                for (int n = 0; n < N; ++n) hT[((size_t)b * dim + d) * N + n] = (float)s[n];
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-1 single-token step — selective_scan_step (mamba1.rs:666-733) with  */
/* the same optional bias/softplus/gate as mamba1_scan.  u,delta,z,y[b,d];   */
/* B,C[b,n]; state[b,d,n] updated in place.                                  */
/* ------------------------------------------------------------------------- */
void F(mamba1_step)(int batch, int dim, int dstate, const float* u, const float* delta,
                    const float* A, const float* B, const float* C, const float* D,
                    const float* z, const float* delta_bias, int delta_softplus, float* state,
                    float* y) {
    const int N = dstate;
    for (int b = 0; b < batch; ++b)
        for (int d = 0; d < dim; ++d) {
            REAL dl = delta[(size_t)b * dim + d];
            if (delta_bias) dl += (REAL)delta_bias[d];
            if (delta_softplus) dl = (REAL)log1p(exp((double)dl));
            const REAL uv = u[(size_t)b * dim + d];
            REAL acc = 0;
            for (int n = 0; n < N; ++n) {
                float* sp = state + ((size_t)b * dim + d) * N + n;
                const REAL a = F(exp_)(dl * (REAL)A[(size_t)d * N + n]);
                const REAL sv = (REAL)*sp * a + (dl * (REAL)B[(size_t)b * N + n]) * uv;
                *sp = (float)sv;
                acc += sv * (REAL)C[(size_t)b * N + n];
            }
            REAL out = acc + (D ? (REAL)D[d] : (REAL)0) * uv;
            if (z) out *= F(silu_)((REAL)z[(size_t)b * dim + d]);
            y[(size_t)b * dim + d] = (float)out;
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-2 block step() — src/mamba2/mamba2.rs:820-1004 — between in_proj and */
/* out_proj: conv-window slide + depthwise dot + bias + SiLU (:865-902),      */
/* split (:907-918), dt = softplus(dt_raw + dt_bias).clamp(lo,hi) (:924),     */
/* dA = exp(dt*A) (:932), h = h*dA + dt*B*x (:940-966), y = sum_n h*C + D*x   */
/* (:970-991), gated RMSNorm (:995, rms_norm_gated.rs:70-135): with          */
/* norm_before_gate = 0 (the default) g = y*silu(z), g/sqrt(mean(g^2)+eps)*w; */
/* with 1, y/sqrt(mean(y^2)+eps)*w*silu(z).                                   */
/*   zxbcdt[b, d_inner + conv_dim + H]  conv_state[b, conv_dim, K] (in/out)   */
/*   conv_w[conv_dim, K] conv_b[conv_dim] (nullable) dt_bias[H] A[H] D[H]     */
/*   norm_w[d_inner]  ssm_state[b,H,P,N] (in/out)  out[b, d_inner]            */
/* ------------------------------------------------------------------------- */
void F(mamba2_step_ssm)(int batch, int nheads, int headdim, int ngroups, int dstate, int conv_k,
                        const float* zxbcdt, float* conv_state, const float* conv_w,
                        const float* conv_b, const float* dt_bias, const float* A, const float* D,
                        float dt_lo, float dt_hi, const float* norm_w, float* ssm_state,
                        float* out, int norm_before_gate) {
    const int H = nheads, P = headdim, G = ngroups, N = dstate, K = conv_k;
    const int d_inner = H * P, conv_dim = d_inner + 2 * G * N, hpg = H / G;
    const int d_in_proj = d_inner + conv_dim + H;
#pragma omp parallel for schedule(static)
    for (int b = 0; b < batch; ++b) {
        REAL* xbc = (REAL*)malloc(sizeof(REAL) * conv_dim);
        REAL* g = (REAL*)malloc(sizeof(REAL) * d_inner);
        const float* row = zxbcdt + (size_t)b * d_in_proj;
        for (int v = 0; v < conv_dim; ++v) {
            float* cw = conv_state + ((size_t)b * conv_dim + v) * K;
            for (int k = 0; k + 1 < K; ++k) cw[k] = cw[k + 1];
            cw[K - 1] = row[d_inner + v];
            REAL acc = 0;
            for (int k = 0; k < K; ++k) acc += (REAL)cw[k] * (REAL)conv_w[(size_t)v * K + k];
            if (conv_b) acc += (REAL)conv_b[v];
            xbc[v] = F(silu_)(acc);
        }
        REAL ssq = 0;
        for (int h = 0; h < H; ++h) {
            const int gi = h / hpg;
            REAL dtv = F(softplus_)((REAL)row[d_inner + conv_dim + h] + (REAL)dt_bias[h]);
            if (dtv < (REAL)dt_lo) dtv = (REAL)dt_lo;
            if (dtv > (REAL)dt_hi) dtv = (REAL)dt_hi;
            const REAL dA = F(exp_)(dtv * (REAL)A[h]);
            const REAL* xh = xbc + (size_t)h * P;
            const REAL* bg = xbc + d_inner + (size_t)gi * N;
            const REAL* cg = xbc + d_inner + (size_t)G * N + (size_t)gi * N;
            for (int p = 0; p < P; ++p) {
                REAL acc = 0;
                for (int n = 0; n < N; ++n) {
                    float* sp = ssm_state + (((size_t)b * H + h) * P + p) * N + n;
                    const REAL sv = (REAL)*sp * dA + (dtv * bg[n]) * xh[p];
                    *sp = (float)sv;
                    acc += sv * cg[n];
                }
                const REAL yv = acc + (D ? (REAL)D[h] : (REAL)0) * xh[p];
                const REAL gv = norm_before_gate ? yv : yv * F(silu_)((REAL)row[(size_t)h * P + p]);
                g[h * P + p] = gv;
                ssq += gv * gv;
            }
        }
        const REAL rms = (REAL)sqrt((double)(ssq / (REAL)d_inner + F(div_eps_)()));
        for (int i = 0; i < d_inner; ++i) {
            REAL v = (g[i] / rms) * (REAL)norm_w[i];
            if (norm_before_gate) v *= F(silu_)((REAL)row[i]);
            out[(size_t)b * d_inner + i] = (float)v;
        }
        free(xbc);
        free(g);
    }
}

/* Depthwise causal conv, one step: the window roll + dot + bias (+ SiLU) of   */
/* Mamba1::step (src/mamba1/mamba1.rs:558-597).  x[b,c]; state[b,c,K] in place;*/
/* w[c,K]; bias[c] (nullable); out[b,c].                                      */
void F(conv1d_step)(int batch, int channels, int K, const float* x, float* state, const float* w,
                    const float* bias, int silu, float* out) {
    for (int b = 0; b < batch; ++b)
        for (int c = 0; c < channels; ++c) {
            float* win = state + ((size_t)b * channels + c) * K;
            for (int k = 0; k + 1 < K; ++k) win[k] = win[k + 1];
            win[K - 1] = x[(size_t)b * channels + c];
            REAL acc = 0;
            for (int k = 0; k < K; ++k) acc += (REAL)win[k] * (REAL)w[(size_t)c * K + k];
            if (bias) acc += (REAL)bias[c];
            out[(size_t)b * channels + c] = (float)(silu ? F(silu_)(acc) : acc);
        }
}

/* RmsNorm (src/modules/norm/rms_norm.rs:53-98): x / sqrt(mean(x^2)+eps) * w. */
void F(rmsnorm)(int rows, int cols, const float* x, const float* w, float* out) {
    for (int r = 0; r < rows; ++r) {
        REAL ssq = 0;
        for (int c = 0; c < cols; ++c) ssq += (REAL)x[(size_t)r * cols + c] * (REAL)x[(size_t)r * cols + c];
        const REAL rms = (REAL)sqrt((double)(ssq / (REAL)cols + F(div_eps_)()));
        for (int c = 0; c < cols; ++c)
            out[(size_t)r * cols + c] = (float)(((REAL)x[(size_t)r * cols + c] / rms) * (REAL)w[c]);
    }
}

/* Dense x[rows,k] @ W[k,cols] (Burn Linear weight layout [d_in, d_out]). */
void F(linear)(int rows, int k, int cols, const float* x, const float* W, const float* bias,
               float* out) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        REAL* acc = (REAL*)calloc(cols, sizeof(REAL));
        for (int i = 0; i < k; ++i) {
            const REAL xv = x[(size_t)r * k + i];
            const float* wr = W + (size_t)i * cols;
            for (int c = 0; c < cols; ++c) acc[c] += xv * (REAL)wr[c];
        }
        for (int c = 0; c < cols; ++c) out[(size_t)r * cols + c] = (float)(acc[c] + (bias ? (REAL)bias[c] : (REAL)0));
        free(acc);
    }
}

/* ------------------------------------------------------------------------- */
/* Mamba-3 single-pass SSD, serial K1..K5 —                                   */
/* src/mamba3/single_ssd/ssd/serial.rs:56-268 with K1-K4 from                 */
/* src/mamba3/double_ssd/ssd/serial.rs:118-286 and the y-diag correction of   */
/* src/mamba3/single_ssd/ssd/diag.rs:50-100.  MIMO rank M is fused into the   */
/* chunk axis as t*M+m (single_ssd/ssd/minimal.rs:152-172).                   */
/*   y_off  = exp(cs_i) * C_i . h_in                                          */
/*   y_low  = sum_{j<i} sum_mi (C_i,mo . B_j,mi) exp(cs_i-cs_j) scale_j v_j,mi */
/*   y_diag = gamma_i sum_mi (C_i,mo . B_i,mi) v_i,mi                          */
/*   S      = sum_{j,mi} exp(cs_end-cs_j) v_j,mi (x) (B_j,mi * scale_j)        */
/* ------------------------------------------------------------------------- */
void F(ssd3_serial)(int batch, int seqlen, int mimo, int nheads, int headdim, int dstate, int chunk,
                    const float* v, const float* da, const float* B, const float* C,
                    const float* gamma, const float* scale, const float* h0, float* y, float* hT) {
    const int M = mimo, H = nheads, P = headdim, N = dstate, Q = chunk;
    const int nch = (seqlen + Q - 1) / Q;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            const size_t PN = (size_t)P * N;
            REAL* cs = (REAL*)calloc((size_t)nch * Q, sizeof(REAL));
            REAL* S = (REAL*)calloc((size_t)nch * PN, sizeof(REAL));
            REAL* hin = (REAL*)calloc((size_t)nch * PN, sizeof(REAL));
            REAL* run = (REAL*)calloc(PN, sizeof(REAL));
#define T_OF(c, l) ((c) * Q + (l))
#define DA(t) ((t) < seqlen ? (REAL)da[((size_t)b * seqlen + (t)) * H + h] : (REAL)0)
#define GM(t) ((t) < seqlen ? (REAL)gamma[((size_t)b * seqlen + (t)) * H + h] : (REAL)0)
#define SC(t) ((t) < seqlen ? (REAL)scale[((size_t)b * seqlen + (t)) * H + h] : (REAL)0)
#define VV(t, m, p) ((t) < seqlen ? (REAL)v[((((size_t)b * seqlen + (t)) * M + (m)) * H + h) * P + (p)] : (REAL)0)
#define BV(t, m, n) ((t) < seqlen ? (REAL)B[((((size_t)b * seqlen + (t)) * M + (m)) * H + h) * N + (n)] : (REAL)0)
#define CV(t, m, n) ((t) < seqlen ? (REAL)C[((((size_t)b * seqlen + (t)) * M + (m)) * H + h) * N + (n)] : (REAL)0)
            for (int c = 0; c < nch; ++c) {
                REAL acc = 0;
                for (int l = 0; l < Q; ++l) { acc += DA(T_OF(c, l)); cs[T_OF(c, l)] = acc; }
            }
            /* K3 with K = B * scale (serial.rs:82-93; double_ssd/ssd/serial.rs:184-220). */
            for (int c = 0; c < nch; ++c) {
                const REAL end = cs[T_OF(c, Q - 1)];
                REAL* Sc = S + (size_t)c * PN;
                for (int l = 0; l < Q; ++l) {
                    const int t = T_OF(c, l);
                    if (t >= seqlen) break;
                    const REAL dec = F(exp_)(end - cs[t]);
                    for (int m = 0; m < M; ++m)
                        for (int p = 0; p < P; ++p) {
                            const REAL dv = dec * VV(t, m, p);
                            for (int n = 0; n < N; ++n) Sc[p * N + n] += dv * (BV(t, m, n) * SC(t));
                        }
                }
            }
            /* K4 (double_ssd/ssd/serial.rs:239-286). */
            for (size_t i = 0; i < PN; ++i) run[i] = h0 ? (REAL)h0[((size_t)b * H + h) * PN + i] : (REAL)0;
            for (int c = 0; c < nch; ++c) {
                const REAL dec = F(exp_)(cs[T_OF(c, Q - 1)]);
                memcpy(hin + (size_t)c * PN, run, sizeof(REAL) * PN);
                for (size_t i = 0; i < PN; ++i) run[i] = dec * run[i] + S[(size_t)c * PN + i];
            }
            for (size_t i = 0; i < PN; ++i) hT[((size_t)b * H + h) * PN + i] = (float)run[i];
            /* K5 single (single_ssd/ssd/serial.rs:156-268); the C.B^T row of each
             * output (K2, computed once per chunk as the reference does) is
             * formed before the headdim loop. */
            REAL* cbrow = (REAL*)malloc(sizeof(REAL) * (size_t)Q * M);
            for (int c = 0; c < nch; ++c) {
                const REAL* hc = hin + (size_t)c * PN;
                for (int i = 0; i < Q; ++i) {
                    const int ti = T_OF(c, i);
                    if (ti >= seqlen) break;
                    for (int mo = 0; mo < M; ++mo) {
                        for (int j = 0; j <= i; ++j)
                            for (int mi = 0; mi < M; ++mi) {
                                REAL cbv = 0;
                                for (int n = 0; n < N; ++n) cbv += CV(ti, mo, n) * BV(T_OF(c, j), mi, n);
                                cbrow[j * M + mi] = cbv;
                            }
                        for (int p = 0; p < P; ++p) {
                            REAL ch = 0;
                            for (int n = 0; n < N; ++n) ch += CV(ti, mo, n) * hc[p * N + n];
                            const REAL yoff = ch * F(exp_)(cs[ti]);
                            REAL ylow = 0;
                            for (int j = 0; j < i; ++j) {
                                const int tj = T_OF(c, j);
                                const REAL ker = F(exp_)(cs[ti] - cs[tj]) * SC(tj);
                                for (int mi = 0; mi < M; ++mi) ylow += (cbrow[j * M + mi] * ker) * VV(tj, mi, p);
                            }
                            REAL ydiag = 0;
                            for (int mi = 0; mi < M; ++mi) ydiag += cbrow[i * M + mi] * VV(ti, mi, p);
                            ydiag *= GM(ti);
                            y[((((size_t)b * seqlen + ti) * M + mo) * H + h) * P + p] = (float)((yoff + ylow) + ydiag);
                        }
                    }
                }
            }
            free(cbrow);
#undef T_OF
#undef DA
#undef GM
#undef SC
#undef VV
#undef BV
#undef CV
            free(cs); free(S); free(hin); free(run);
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-3 merged-form recurrence, token by token: the single-SSD accumulator */
/*   y_t,mo = C_t,mo . (alpha_t h') + gamma_t sum_mi (C_t,mo.B_t,mi) v_t,mi    */
/*   h'     = alpha_t h' + scale_t sum_mi v_t,mi (x) B_t,mi                    */
/* with alpha_t = exp(da_t) — the sequential form the chunked single-SSD      */
/* computes (single_ssd/ssd/ssd_path/mod.rs:20-27; single_ssd/mod.rs:1-13).   */
/* ------------------------------------------------------------------------- */
void F(ssd3_recurrent)(int batch, int seqlen, int mimo, int nheads, int headdim, int dstate,
                       const float* v, const float* da, const float* B, const float* C,
                       const float* gamma, const float* scale, const float* h0, float* y,
                       float* hT) {
    const int M = mimo, H = nheads, P = headdim, N = dstate;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            const size_t PN = (size_t)P * N;
            REAL* s = (REAL*)calloc(PN, sizeof(REAL));
            for (size_t i = 0; i < PN; ++i) s[i] = h0 ? (REAL)h0[((size_t)b * H + h) * PN + i] : (REAL)0;
            for (int t = 0; t < seqlen; ++t) {
                const size_t bt = (size_t)b * seqlen + t;
                const REAL al = F(exp_)((REAL)da[bt * H + h]);
                const REAL gm = gamma[bt * H + h], sc = scale[bt * H + h];
                for (size_t i = 0; i < PN; ++i) s[i] *= al;
                for (int mo = 0; mo < M; ++mo) {
                    const float* cr = C + ((bt * M + mo) * H + h) * N;
                    for (int p = 0; p < P; ++p) {
                        REAL acc = 0;
                        for (int n = 0; n < N; ++n) acc += (REAL)cr[n] * s[p * N + n];
                        REAL dg = 0;
                        for (int mi = 0; mi < M; ++mi) {
                            const float* br = B + ((bt * M + mi) * H + h) * N;
                            REAL qk = 0;
                            for (int n = 0; n < N; ++n) qk += (REAL)cr[n] * (REAL)br[n];
                            dg += qk * (REAL)v[((bt * M + mi) * H + h) * P + p];
                        }
                        y[((bt * M + mo) * H + h) * P + p] = (float)(acc + gm * dg);
                    }
                }
                for (int mi = 0; mi < M; ++mi) {
                    const float* br = B + ((bt * M + mi) * H + h) * N;
                    const float* vr = v + ((bt * M + mi) * H + h) * P;
                    for (int p = 0; p < P; ++p)
                        for (int n = 0; n < N; ++n) s[p * N + n] += sc * ((REAL)vr[p] * (REAL)br[n]);
                }
            }
            for (size_t i = 0; i < PN; ++i) hT[((size_t)b * H + h) * PN + i] = (float)s[i];
            free(s);
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-3 per-token prep — Mamba3::step_project (src/mamba3/double_ssd/      */
/* double_ssd/mod.rs:407-496) and rotate_bc_step for Complex2D                 */
/* (src/mamba3/rotation/mod.rs:729-763).  The in_proj row splits as           */
/* [z | x | b_raw (M,G,N) | c_raw (M,G,N) | dd_dt (H) | dd_a (H) | lambda (H) | */
/*  rot (A)] (:430-447), A = max(rope_dim/2, 1) angles (mamba3.rs:565-567).   */
/* trapezoidal_coefficients (helpers.rs:42-73):                               */
/*   dt = clamp(softplus(dd_dt + dt_bias)), a = -max(softplus(dd_a), a_floor), */
/*   alpha = exp(dt a), beta = (1 - sigmoid(lambda)) dt alpha,                */
/*   gamma = sigmoid(lambda) dt.                                              */
/* qk_norm_expand_bias (helpers.rs:82-95): RmsNorm over N, group h/(H/G),     */
/* + bias[h,m,n].  angle_increment (rotation/mod.rs:559-567):                 */
/*   angle[b,h,a] = wrap(angle + dt range pi tanh(rot[a])), wrap_angle        */
/* (rope.rs:23-27) subtracting round(x / 2pi) 2pi; apply_rope_partial         */
/* (rope.rs:118-170): pairs (2a, 2a+1) when M == 1, (a, a + N/2) otherwise,   */
/* for a < rope_dim/2; rope_dim == 0 rotates nothing.                          */
/*   proj[b, *]; angle[b,H,A] in/out; Bo, Co[b,M,H,N]; dt/alpha/beta/gamma[b,H] */
/* ------------------------------------------------------------------------- */
static inline REAL F(wrap_)(REAL a) {
    const REAL two_pi = (REAL)(2.0f * 3.14159265358979323846f);
    const REAL k = (REAL)nearbyint((double)(a * ((REAL)1 / two_pi)));
    return a - k * two_pi;
}

void F(mamba3_step_prep)(int batch, int nheads, int headdim, int ngroups, int dstate, int mimo,
                         int rope_dim, const float* proj, const float* dt_bias, float a_floor,
                         float dt_lo, float dt_hi, float rot_range, const float* b_norm_w,
                         const float* c_norm_w, const float* b_bias, const float* c_bias,
                         float* angle, float* Bo, float* Co, float* dt_o, float* alpha_o,
                         float* beta_o, float* gamma_o) {
    const int H = nheads, P = headdim, G = ngroups, N = dstate, M = mimo, hpg = H / G;
    const int A = rope_dim / 2 > 1 ? rope_dim / 2 : 1;
    const int d_inner = H * P, bc = M * G * N;
    const size_t row_len = (size_t)2 * d_inner + 2 * bc + 3 * H + A;
    const REAL span = (REAL)((double)rot_range * 3.14159265358979323846);  /* range * pi */
    for (int b = 0; b < batch; ++b) {
        const float* row = proj + (size_t)b * row_len;
        const float* braw = row + 2 * d_inner;
        const float* craw = braw + bc;
        const float* dd_dt = craw + bc;
        const float* dd_a = dd_dt + H;
        const float* lam = dd_a + H;
        const float* rot = lam + H;
        for (int h = 0; h < H; ++h) {
            REAL dt = F(softplus_)((REAL)dd_dt[h] + (REAL)dt_bias[h]);
            if (dt < (REAL)dt_lo) dt = (REAL)dt_lo;
            if (dt > (REAL)dt_hi) dt = (REAL)dt_hi;
            REAL sa = F(softplus_)((REAL)dd_a[h]);
            if (sa < (REAL)a_floor) sa = (REAL)a_floor;
            const REAL a = -sa;
            const REAL l = (REAL)1 / ((REAL)1 + F(exp_)(-(REAL)lam[h]));
            const REAL al = F(exp_)(dt * a);
            const size_t bh = (size_t)b * H + h;
            dt_o[bh] = (float)dt;
            alpha_o[bh] = (float)al;
            beta_o[bh] = (float)(((REAL)1 - l) * dt * al);
            gamma_o[bh] = (float)(l * dt);
            /* cumulative angle of this head */
            float* ang = angle + bh * A;
            for (int k = 0; k < A; ++k) {
                const REAL inc = dt * ((REAL)tanh((double)rot[k]) * span);
                ang[k] = (float)F(wrap_)((REAL)ang[k] + inc);
            }
            const int g = h / hpg;
            for (int m = 0; m < M; ++m)
                for (int which = 0; which < 2; ++which) {
                    const float* src = (which ? craw : braw) + ((size_t)m * G + g) * N;
                    const float* nw = which ? c_norm_w : b_norm_w;
                    const float* bias = (which ? c_bias : b_bias) + ((size_t)h * M + m) * N;
                    float* dst = (which ? Co : Bo) + (((size_t)b * M + m) * H + h) * N;
                    REAL ssq = 0;
                    for (int n = 0; n < N; ++n) ssq += (REAL)src[n] * (REAL)src[n];
                    const REAL rms = (REAL)sqrt((double)(ssq / (REAL)N + F(div_eps_)()));
                    REAL* tmp = (REAL*)malloc(sizeof(REAL) * N);
                    for (int n = 0; n < N; ++n) tmp[n] = ((REAL)src[n] / rms) * (REAL)nw[n] + (REAL)bias[n];
                    if (rope_dim > 0)
                        for (int k = 0; k < rope_dim / 2; ++k) {
                            const int i0 = M == 1 ? 2 * k : k, i1 = M == 1 ? 2 * k + 1 : k + N / 2;
                            const REAL th = F(wrap_)((REAL)ang[k]);
                            const REAL cs = (REAL)cos((double)th), sn = (REAL)sin((double)th);
                            const REAL x0 = tmp[i0], x1 = tmp[i1];
                            tmp[i0] = cs * x0 - sn * x1;
                            tmp[i1] = sn * x0 + cs * x1;
                        }
                    for (int n = 0; n < N; ++n) dst[n] = (float)tmp[n];
                    free(tmp);
                }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Mamba-3 token state update + readout — Mamba3::step_double_ssd             */
/* (src/mamba3/double_ssd/double_ssd/mod.rs:699-733), build_v_with_mimo       */
/* (helpers.rs:152-168), mimo_outer_sum (:113-140), step_readout (mod.rs:516-  */
/* 550) and the D skip of step_finish (:565-573):                             */
/*   v[m,p] = x[p] mimo_x[h,m,p]      xs[m,p] = v_state[p] mimo_x[h,m,p]      */
/*   h      = alpha h + sum_m gamma v[m] (x) B[m] + sum_m beta xs[m] (x) K[m]  */
/*   out    = sum_n C[m,n] h[p,n] + D v[m,p]                                  */
/* mimo_x NULL means M == 1 with v = x.  x, v_state[b,H,P]; B, K, C[b,M,H,N];  */
/* alpha/beta/gamma[b,H]; state[b,H,P,N] in/out; out[b,M,H,P].                */
/* ------------------------------------------------------------------------- */
void F(mamba3_step_core)(int batch, int nheads, int headdim, int dstate, int mimo, const float* x,
                         const float* v_state, const float* Bm, const float* K, const float* Cm,
                         const float* alpha, const float* beta, const float* gamma,
                         const float* mimo_x, const float* D, float* state, float* out) {
    const int H = nheads, P = headdim, N = dstate, M = mimo;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            const size_t bh = (size_t)b * H + h;
            const REAL al = alpha[bh], be = beta[bh], ga = gamma[bh];
            REAL* v = (REAL*)malloc(sizeof(REAL) * M * P);
            REAL* xs = (REAL*)malloc(sizeof(REAL) * M * P);
            for (int m = 0; m < M; ++m)
                for (int p = 0; p < P; ++p) {
                    const REAL mx = mimo_x ? (REAL)mimo_x[((size_t)h * M + m) * P + p] : (REAL)1;
                    v[m * P + p] = (REAL)x[bh * P + p] * mx;
                    xs[m * P + p] = (REAL)v_state[bh * P + p] * mx;
                }
            for (int p = 0; p < P; ++p) {
                float* sp = state + (bh * P + p) * N;
                for (int n = 0; n < N; ++n) {
                    REAL acc = al * (REAL)sp[n];
                    for (int m = 0; m < M; ++m) {
                        const size_t bi = (((size_t)b * M + m) * H + h) * N + n;
                        acc += (ga * v[m * P + p]) * (REAL)Bm[bi] + (be * xs[m * P + p]) * (REAL)K[bi];
                    }
                    sp[n] = (float)acc;
                }
                for (int m = 0; m < M; ++m) {
                    const float* cr = Cm + (((size_t)b * M + m) * H + h) * N;
                    REAL acc = 0;
                    for (int n = 0; n < N; ++n) acc += (REAL)cr[n] * (REAL)sp[n];
                    out[(((size_t)b * M + m) * H + h) * P + p] =
                        (float)(acc + (D ? (REAL)D[h] : (REAL)0) * v[m * P + p]);
                }
            }
            free(v);
            free(xs);
        }
}

/* ------------------------------------------------------------------------- */
/* Mamba-3 step_finish without out_proj (double_ssd/double_ssd/mod.rs:556-628):*/
/*   M > 1: y[p] = sum_m mimo_o[h,m,p] G(out[m,p], z[p] mimo_z[h,m,p])         */
/*   M = 1: y[p] = G(out[0,p], z[p])                                          */
/* G(y, z) = y silu(z), or with norm_w (has_outproj_norm, RmsNormGated with   */
/* norm_before_gate = true over the P entries of one (m, head), mamba3.rs:744- */
/* 748, rms_norm_gated.rs:70-135): y / sqrt(mean_p(y^2) + eps) w[p] silu(z).  */
/* out[b,M,H,P]; z[b,H*P]; y[b,H*P].                                          */
/* ------------------------------------------------------------------------- */
void F(mamba3_step_finish)(int batch, int nheads, int headdim, int mimo, const float* out,
                           const float* z, const float* mimo_z, const float* mimo_o,
                           const float* norm_w, float* y) {
    const int H = nheads, P = headdim, M = mimo;
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < H; ++h) {
            REAL* acc = (REAL*)calloc(P, sizeof(REAL));
            for (int m = 0; m < M; ++m) {
                const float* o = out + (((size_t)b * M + m) * H + h) * P;
                REAL rms = 1;
                if (norm_w) {
                    REAL ssq = 0;
                    for (int p = 0; p < P; ++p) ssq += (REAL)o[p] * (REAL)o[p];
                    rms = (REAL)sqrt((double)(ssq / (REAL)P + F(div_eps_)()));
                }
                for (int p = 0; p < P; ++p) {
                    REAL zv = (REAL)z[((size_t)b * H + h) * P + p];
                    if (M > 1) zv *= (REAL)mimo_z[((size_t)h * M + m) * P + p];
                    REAL gv = norm_w ? ((REAL)o[p] / rms) * (REAL)norm_w[p] * F(silu_)(zv)
                                     : (REAL)o[p] * F(silu_)(zv);
                    if (M > 1) gv *= (REAL)mimo_o[((size_t)h * M + m) * P + p];
                    acc[p] += gv;
                }
            }
            for (int p = 0; p < P; ++p) y[((size_t)b * H + h) * P + p] = (float)acc[p];
            free(acc);
        }
}

#undef F
#undef CAT
#undef CAT2
