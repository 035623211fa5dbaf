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

extern "C" int mamba_ssd2_bwd(const mamba_ssd2_bwd_args* a, void* workspace, size_t workspace_bytes,
                              mamba_stream_t stream) {
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
    // dynamic LDS above the 64 KB default (up to the CU's 160 KB)
    MAMBA_CHECK_HIP(hipFuncSetAttribute((const void*)ssd2_bwd_states, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)bwd_states_lds(p.P, p.N)));
    MAMBA_CHECK_HIP(hipFuncSetAttribute((const void*)ssd2_bwd_chunks, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)bwd_chunks_lds(p.P, p.N)));
    hipLaunchKernelGGL(ssd2_bwd_states, grid, dim3(kBwdT), bwd_states_lds(p.P, p.N), s, p);
    MAMBA_CHECK_LAUNCH();
    hipLaunchKernelGGL(ssd2_bwd_chunks, grid, dim3(kBwdT), bwd_chunks_lds(p.P, p.N), s, p);
    MAMBA_CHECK_LAUNCH();
    const int64_t fin = a->ngroups == a->nheads ? 0 : (int64_t)a->batch * a->seqlen * a->ngroups * a->dstate;
    const int fgrid = (int)std::max<int64_t>((a->nheads + 255) / 256, std::min<int64_t>((fin + 255) / 256, 4096));
    hipLaunchKernelGGL(ssd2_bwd_finish, dim3(fgrid), dim3(256), 0, s, p, a->dA, a->dD, a->dB, a->dC);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}
