// Mamba-3 single-pass ("single-SSD") chunked SSD forward for gfx950.
//
// Reference: Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated
// (burn-mamba src/mamba3/single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-164):
// K1 cumsum of da, K2 C.B^T on the fused (time, mimo) axis, K3 chunk state on
// scale * B, K4 state passing (double_ssd/ssd/serial.rs:118-286) and the
// single-SSD K5 (:192-291) with its gamma same-step correction
// (single_ssd/ssd/diag.rs:50-100).  For output step t, MIMO row mo:
//
//   y[t,mo,:] = exp(cs_t) C[t,mo].h_in
//             + sum_{t' < t, mi} (C[t,mo].B[t',mi]) exp(cs_t - cs_t') scale_t' v[t',mi,:]
//             + gamma_t sum_mi (C[t,mo].B[t,mi]) v[t,mi,:]
//   h_out     = exp(cs_end) h_in + sum_{t, mi} exp(cs_end - cs_t) scale_t v[t,mi,:] (x) B[t,mi,:]
//
// cs is the within-chunk cumulative sum of da (= dt A); positions past seqlen
// read as zero.  This file holds the shape-generic path: three SIMT kernels
// (chunk state, state passing, chunk scan) with f32 arithmetic and f32 or bf16
// I/O; chunk_len counts base time steps.  bf16 calls with headdim 64, dstate
// 128 and a MIMO rank dividing 32 take the single-kernel MFMA path
// (ssd3_mfma.hip), which chunks on 128 fused positions whatever chunk_len
// says: the chunked form is exact for any chunk length, so only rounding
// differs.
#include "common.h"

namespace mamba {

struct Ssd3Params {
    int nb, L, M, H, P, G, N, Q, nch;
    int io_dtype;
    const void* v; int64_t v_sb, v_sl, v_sm, v_sh;
    const float* da; int64_t da_sb, da_sl, da_sh;
    const float* gm; int64_t gm_sb, gm_sl, gm_sh;
    const float* sc; int64_t sc_sb, sc_sl, sc_sh;
    const void* Bm; int64_t B_sb, B_sl, B_sm, B_sg;
    const void* Cm; int64_t C_sb, C_sl, C_sm, C_sg;
    const float* h0;
    void* y; int64_t y_sb, y_sl, y_sm, y_sh;
    float* hT;
};

__device__ __forceinline__ float ld_io(const void* base, int64_t i, bool bf16) {
    return bf16 ? bf16_to_f32(static_cast<const bf16_t*>(base)[i]) : static_cast<const float*>(base)[i];
}

// cs[l] = sum_{l' <= l} da over the chunk's base steps; also scale and gamma
// tables.  Steps past seqlen contribute da = scale = gamma = 0.
__device__ void ssd3_chunk_tables(const Ssd3Params& p, int b, int c, int h, float* cs, float* scl, float* gmm,
                                  float* sh4) {
    float carry = 0.f;
    for (int base = 0; base < p.Q; base += 256) {
        const int l = base + threadIdx.x;
        const int t = c * p.Q + l;
        const bool ok = l < p.Q && t < p.L;
        const float dav = ok ? p.da[(int64_t)b * p.da_sb + (int64_t)t * p.da_sl + (int64_t)h * p.da_sh] : 0.f;
        // inclusive block scan of 256 values
        const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
        float v = wave_incl_scan(dav);
        if (lane == 63) sh4[wid] = v;
        __syncthreads();
        float off = 0.f;
        for (int w = 0; w < wid; ++w) off += sh4[w];
        __syncthreads();
        if (l < p.Q) {
            cs[l] = v + off + carry;
            // NULL scale / gamma: unit coefficients (the double-SSD seam)
            scl[l] = !ok ? 0.f : p.sc ? p.sc[(int64_t)b * p.sc_sb + (int64_t)t * p.sc_sl + (int64_t)h * p.sc_sh] : 1.f;
            gmm[l] = !ok ? 0.f : p.gm ? p.gm[(int64_t)b * p.gm_sb + (int64_t)t * p.gm_sl + (int64_t)h * p.gm_sh] : 1.f;
        }
        __syncthreads();
        carry = cs[min(base + 256, p.Q) - 1];
        __syncthreads();
    }
}

// ------------------------------------------------------------ K1 + K3 --
// S[b,c,h,p,n] = sum_{l, m} v[l,m,p] * B[l,m,n] * scale_l * exp(cs_end - cs_l)
// One workgroup per (head, chunk x slice of 256 OPT state entries, batch),
// OPT entries per thread: the launch takes OPT = 4 when (head, chunk, batch)
// alone would give few workgroups (short sequences: more workgroups hide the
// LDS and memory latency of each), else 32 (each slice stages the chunk's v
// and weighted B rows once, so fewer slices stage less).
template <int OPT>
__global__ __launch_bounds__(256) void ssd3_chunk_state_generic(Ssd3Params p, float* states, float* da_end) {
    extern __shared__ float smem[];
    const int nslice = (p.P * p.N + 256 * OPT - 1) / (256 * OPT);
    const int h = blockIdx.x, c = blockIdx.y / nslice, slice = blockIdx.y % nslice, b = blockIdx.z;
    const int g = h / (p.H / p.G);
    const int Q = p.Q, P = p.P, N = p.N, M = p.M;
    const bool bf = p.io_dtype == MAMBA_BF16;
    float* cs = smem;
    float* scl = cs + Q;
    float* gmm = scl + Q;
    float* sh4 = gmm + Q;
    constexpr int TL = 16;  // fused rows staged per pass
    float* vt = sh4 + 4;    // [TL][P]
    float* bt = vt + TL * P;  // [TL][N]
    ssd3_chunk_tables(p, b, c, h, cs, scl, gmm, sh4);
    const float cs_end = cs[Q - 1];
    if (threadIdx.x == 0 && slice == 0) da_end[((int64_t)b * p.H + h) * p.nch + c] = cs_end;
    float* Sout = states + (((int64_t)b * p.nch + c) * p.H + h) * P * N;
    const int QM = Q * M;
    {
        const int e0 = slice * 256 * OPT;
        float acc[OPT];
#pragma unroll
        for (int k = 0; k < OPT; ++k) acc[k] = 0.f;
        for (int f0 = 0; f0 < QM; f0 += TL) {
            __syncthreads();
            for (int i = threadIdx.x; i < TL * P; i += 256) {
                const int f = f0 + i / P, pp = i % P, l = f / M, m = f % M, t = c * Q + l;
                vt[i] = (f < QM && t < p.L)
                            ? ld_io(p.v, (int64_t)b * p.v_sb + (int64_t)t * p.v_sl + (int64_t)m * p.v_sm +
                                             (int64_t)h * p.v_sh + pp, bf)
                            : 0.f;
            }
            for (int i = threadIdx.x; i < TL * N; i += 256) {
                const int f = f0 + i / N, n = i % N, l = f / M, m = f % M, t = c * Q + l;
                float w = 0.f;
                if (f < QM && t < p.L) {
                    const float k = __expf(cs_end - cs[l]) * scl[l];
                    w = ld_io(p.Bm, (int64_t)b * p.B_sb + (int64_t)t * p.B_sl + (int64_t)m * p.B_sm +
                                        (int64_t)g * p.B_sg + n, bf) * k;
                }
                bt[i] = w;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < OPT; ++k) {
                const int e = e0 + k * 256 + threadIdx.x;
                if (e < P * N) {
                    const int pp = e / N, n = e % N;
                    float a = acc[k];
                    for (int r = 0; r < TL; ++r) a += vt[r * P + pp] * bt[r * N + n];
                    acc[k] = a;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < OPT; ++k) {
            const int e = e0 + k * 256 + threadIdx.x;
            if (e < P * N) Sout[e] = acc[k];
        }
    }
}

// ------------------------------------------------------------------ K4 --
__global__ __launch_bounds__(256) void ssd3_state_pass_generic(Ssd3Params p, float* states, const float* da_end) {
    const int h = blockIdx.y, b = blockIdx.z;
    const int PN = p.P * p.N;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= PN) return;
    float run = p.h0 ? p.h0[((int64_t)b * p.H + h) * PN + e] : 0.f;
    const float* de = da_end + ((int64_t)b * p.H + h) * p.nch;
    for (int c = 0; c < p.nch; ++c) {
        float* s = states + (((int64_t)b * p.nch + c) * p.H + h) * PN + e;
        const float tmp = *s;
        *s = run;
        run = __expf(de[c]) * run + tmp;
    }
    p.hT[((int64_t)b * p.H + h) * PN + e] = run;
}

// ------------------------------------------------------------ K2 + K5 --
// One workgroup per (head, chunk x row pass, batch), R fused output rows per pass:
//   y[i][p] = exp(cs_i) C_i.h_in[p] + sum_{j <= i} W[i][j] v[j][p],
//   W[i][j] = (C_i.B_j) scale_j exp(cs_i - cs_j) for step(j) < step(i),
//             (C_i.B_j) gamma_i for step(j) == step(i), 0 after.
// The pass first forms its rows of W in LDS (one exp per (row, source)), then
// thread (column p, row slot rs) accumulates RR rows of one column, so that
// each v[j][p] it loads serves all of them.  The chunk's B rows and the entry
// state are staged in LDS when they fit (flags from the host).
struct Ssd3ScanLds {
    int R, RR, TP;       // rows per pass, rows per thread, row slots (256 / P)
    bool h_lds;          // h_in staged in LDS
};
constexpr int kSsd3BT = 32;  // B rows staged per step of the W product

__global__ __launch_bounds__(256) void ssd3_chunk_scan_generic(Ssd3Params p, const float* states, Ssd3ScanLds ly) {
    extern __shared__ float smem[];
    const int npass = (p.Q * p.M + ly.R - 1) / ly.R;
    const int h = blockIdx.x, c = blockIdx.y / npass, pass = blockIdx.y % npass, b = blockIdx.z;
    const int g = h / (p.H / p.G);
    const int Q = p.Q, P = p.P, N = p.N, M = p.M;
    const bool bf = p.io_dtype == MAMBA_BF16;
    const int QM = Q * M, R = ly.R, RR = ly.RR, TP = ly.TP;
    float* cs = smem;
    float* scl = cs + Q;
    float* gmm = scl + Q;
    float* sh4 = gmm + Q;
    float* W = sh4 + 4;              // [R][QM]
    float* Cs = W + R * QM;          // [R][N]
    const int NB = N + 1;            // Bt row pitch: consecutive sources on different banks
    float* Bt = Cs + R * N;          // [kSsd3BT][NB]: B rows of one step of the W product
    float* Hs = Bt + kSsd3BT * NB;   // [N][P] (h_lds)
    ssd3_chunk_tables(p, b, c, h, cs, scl, gmm, sh4);
    const float* hin = states + (((int64_t)b * p.nch + c) * p.H + h) * P * N;
    const int qvalid = min(Q, p.L - c * Q);
    const int fvalid = qvalid * M;
    auto cptr = [&](int t, int m) { return (int64_t)b * p.C_sb + (int64_t)t * p.C_sl + (int64_t)m * p.C_sm + (int64_t)g * p.C_sg; };
    auto bptr = [&](int t, int m) { return (int64_t)b * p.B_sb + (int64_t)t * p.B_sl + (int64_t)m * p.B_sm + (int64_t)g * p.B_sg; };
    if (ly.h_lds)
        for (int k = threadIdx.x; k < P * N; k += 256) {
            const int pp = k / N, n = k % N;
            Hs[n * P + pp] = hin[k];
        }
    const int pp = threadIdx.x % P, rs = threadIdx.x / P;
    const bool active = rs < TP;
    {
        const int f0 = pass * R;
        if (f0 >= fvalid) return;  // a pass past the chunk's end (the last chunk): nothing to write
        __syncthreads();
        // the pass's C rows
        for (int k = threadIdx.x; k < R * N; k += 256) {
            const int fi = f0 + k / N;
            Cs[k] = fi < fvalid ? ld_io(p.Cm, cptr(c * Q + fi / M, fi % M) + k % N, bf) : 0.f;
        }
        __syncthreads();
        // its rows of W, weights folded in (sources up to the last row's
        // step), kSsd3BT sources at a time: their B rows staged with coalesced
        // loads, then one (row, source) dot per thread
        const int li_last = (min(f0 + R, fvalid) - 1) / M;
        const int nsrc = (li_last + 1) * M;
        for (int s0 = 0; s0 < nsrc; s0 += kSsd3BT) {
            for (int k = threadIdx.x; k < kSsd3BT * N; k += 256) {
                const int j = k / N, n = k % N, fj = s0 + j;
                Bt[j * NB + n] = fj < nsrc ? ld_io(p.Bm, bptr(c * Q + fj / M, fj % M) + n, bf) : 0.f;
            }
            __syncthreads();
            for (int k = threadIdx.x; k < R * kSsd3BT; k += 256) {
                const int r = k / kSsd3BT, j = k % kSsd3BT, fj = s0 + j, fi = f0 + r;
                if (fj >= nsrc) continue;
                const int li = fi / M, lj = fj / M;
                float v = 0.f;
                if (fi < fvalid && lj <= li) {
                    const float* cr = Cs + r * N;
                    const float* br = Bt + j * NB;
                    // four independent partial sums: four LDS loads in flight
                    float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
                    int n = 0;
                    for (; n + 4 <= N; n += 4) {
                        d0 = __builtin_fmaf(cr[n], br[n], d0);
                        d1 = __builtin_fmaf(cr[n + 1], br[n + 1], d1);
                        d2 = __builtin_fmaf(cr[n + 2], br[n + 2], d2);
                        d3 = __builtin_fmaf(cr[n + 3], br[n + 3], d3);
                    }
                    for (; n < N; ++n) d0 = __builtin_fmaf(cr[n], br[n], d0);
                    const float dot = (d0 + d1) + (d2 + d3);
                    v = dot * (lj < li ? __expf(cs[li] - cs[lj]) * scl[lj] : gmm[li]);
                }
                W[r * QM + fj] = v;
            }
            __syncthreads();
        }
        if (!active) return;
        // RR rows of column pp per thread: rows f0 + rs + TP k
        float acc[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = 0.f;
        // sources in groups of 16: their v loads are issued together
        constexpr int U = 16;
        for (int fj0 = 0; fj0 < nsrc; fj0 += U) {
            float vv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int fj = min(fj0 + u, nsrc - 1);  // clamped: its W entries below are skipped
                vv[u] = ld_io(p.v, (int64_t)b * p.v_sb + (int64_t)(c * Q + fj / M) * p.v_sl +
                                       (int64_t)(fj % M) * p.v_sm + (int64_t)h * p.v_sh + pp, bf);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (fj0 + u >= nsrc) break;
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if (k < RR) acc[k] = __builtin_fmaf(W[(rs + TP * k) * QM + fj0 + u], vv[u], acc[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            if (k >= RR) break;
            const int r = rs + TP * k, fi = f0 + r;
            if (fi >= fvalid) continue;
            const int li = fi / M, mo = fi % M, ti = c * Q + li;
            const float* cr = Cs + r * N;
            float b0 = 0.f, b1 = 0.f;
            int n = 0;
            if (ly.h_lds) {
                for (; n + 2 <= N; n += 2) {
                    b0 = __builtin_fmaf(cr[n], Hs[n * P + pp], b0);
                    b1 = __builtin_fmaf(cr[n + 1], Hs[(n + 1) * P + pp], b1);
                }
                for (; n < N; ++n) b0 = __builtin_fmaf(cr[n], Hs[n * P + pp], b0);
            } else {
                for (; n + 2 <= N; n += 2) {
                    b0 = __builtin_fmaf(cr[n], hin[pp * N + n], b0);
                    b1 = __builtin_fmaf(cr[n + 1], hin[pp * N + n + 1], b1);
                }
                for (; n < N; ++n) b0 = __builtin_fmaf(cr[n], hin[pp * N + n], b0);
            }
            const float blue = b0 + b1;
            const float out = __builtin_fmaf(blue, __expf(cs[li]), acc[k]);
            const int64_t yi = (int64_t)b * p.y_sb + (int64_t)ti * p.y_sl + (int64_t)mo * p.y_sm + (int64_t)h * p.y_sh + pp;
            if (bf)
                static_cast<bf16_t*>(p.y)[yi] = f32_to_bf16(out);
            else
                static_cast<float*>(p.y)[yi] = out;
        }
    }
}

// The pass geometry and LDS staging of the chunk scan for these shapes, and
// its dynamic LDS bytes (0 when even the unstaged form does not fit).
static size_t ssd3_scan_layout(const Ssd3Params& p, Ssd3ScanLds* ly, size_t limit_bytes) {
    const int TP = p.P >= 256 ? 1 : 256 / p.P;
    const size_t QM = (size_t)p.Q * p.M;
    const size_t limit = limit_bytes / 4;  // words
    const size_t fixed = 3 * (size_t)p.Q + 4 + (size_t)kSsd3BT * (p.N + 1);
    // rows per thread: up to 16 rows per pass, fewer where the W rows would not fit
    int RR = TP >= 16 ? 1 : 16 / TP;
    while (RR > 1 && fixed + (size_t)TP * RR * (QM + p.N) > limit) RR /= 2;
    ly->TP = TP; ly->RR = RR; ly->R = TP * RR;
    size_t words = fixed + (size_t)ly->R * (QM + p.N);
    if (words > limit) return 0;
    ly->h_lds = words + (size_t)p.P * p.N <= limit;
    if (ly->h_lds) words += (size_t)p.P * p.N;
    return words * 4;
}

// ------------------------------------------------------------ host side --
// unit: the double-SSD seam, whose gamma and scale are NULL (unit coefficients)
static int ssd3_make_params(const mamba_ssd3_args* a, Ssd3Params* out, bool unit = false) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->mimo > 0, "batch, seqlen and mimo must be >= 1");
    MAMBA_CHECK_ARG(a->nheads > 0 && a->headdim > 0 && a->dstate > 0, "nheads/headdim/dstate must be >= 1");
    MAMBA_CHECK_ARG(a->headdim <= 256 && a->dstate <= 256 && a->mimo <= 64, "headdim, dstate <= 256, mimo <= 64");
    MAMBA_CHECK_ARG(a->ngroups > 0 && a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    MAMBA_CHECK_ARG(a->chunk_len > 0 && a->chunk_len * a->mimo <= 4096, "chunk_len * mimo must be in [1, 4096]");
    MAMBA_CHECK_ARG(a->io_dtype == MAMBA_F32 || a->io_dtype == MAMBA_BF16, "io_dtype must be MAMBA_F32 or MAMBA_BF16");
    MAMBA_CHECK_ARG(a->v && a->da && a->B && a->C && a->y && a->final_state,
                    "v, da, B, C, y and final_state are required");
    MAMBA_CHECK_ARG(unit ? (a->gamma == nullptr && a->scale == nullptr) : (a->gamma && a->scale),
                    "gamma and scale are required");
    Ssd3Params& p = *out;
    p.nb = a->batch; p.L = a->seqlen; p.M = a->mimo; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups;
    p.N = a->dstate; p.Q = a->chunk_len; p.nch = (a->seqlen + a->chunk_len - 1) / a->chunk_len;
    p.io_dtype = a->io_dtype;
    p.v = a->v; p.v_sb = a->v_sb; p.v_sl = a->v_sl; p.v_sm = a->v_sm; p.v_sh = a->v_sh;
    p.da = a->da; p.da_sb = a->da_sb; p.da_sl = a->da_sl; p.da_sh = a->da_sh;
    p.gm = a->gamma; p.gm_sb = a->gamma_sb; p.gm_sl = a->gamma_sl; p.gm_sh = a->gamma_sh;
    p.sc = a->scale; p.sc_sb = a->scale_sb; p.sc_sl = a->scale_sl; p.sc_sh = a->scale_sh;
    p.Bm = a->B; p.B_sb = a->B_sb; p.B_sl = a->B_sl; p.B_sm = a->B_sm; p.B_sg = a->B_sg;
    p.Cm = a->C; p.C_sb = a->C_sb; p.C_sl = a->C_sl; p.C_sm = a->C_sm; p.C_sg = a->C_sg;
    p.h0 = a->initial_state;
    p.y = a->y; p.y_sb = a->y_sb; p.y_sl = a->y_sl; p.y_sm = a->y_sm; p.y_sh = a->y_sh;
    p.hT = a->final_state;
    return MAMBA_OK;
}

static size_t ssd3_ws_bytes(const Ssd3Params& p) {
    return align_up((size_t)p.nb * p.nch * p.H * p.P * p.N * 4, 256) + align_up((size_t)p.nb * p.H * p.nch * 4, 256);
}

bool ssd3_mfma_supported(const mamba_ssd3_args* a);
int ssd3_mfma_launch(const mamba_ssd3_args* a, hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1);

static int ssd3_dispatch(const mamba_ssd3_args* a, void* ws, size_t ws_bytes, hipStream_t stream, hipEvent_t ev0,
                         hipEvent_t ev1, bool allow_fast, bool unit = false) {
    Ssd3Params p;
    int st = ssd3_make_params(a, &p, unit);
    if (st != MAMBA_OK) return st;
    if (allow_fast && ssd3_mfma_supported(a)) return ssd3_mfma_launch(a, stream, ev0, ev1);
    const size_t need = ssd3_ws_bytes(p);
    if (ws == nullptr || ws_bytes < need) {
        set_error("mamba_ssd3_fwd: workspace of " + std::to_string(need) + " bytes required");
        return MAMBA_ERR_WORKSPACE;
    }
    Ssd3ScanLds ly;
    const size_t sm_state = (3 * (size_t)p.Q + 4 + 16 * (size_t)p.P + 16 * (size_t)p.N) * 4;
    const size_t sm_scan = ssd3_scan_layout(p, &ly, 64 * 1024);
    MAMBA_CHECK_ARG(sm_scan > 0 && sm_state <= 160 * 1024, "chunk_len * mimo too large for the generic path");
    float* states = static_cast<float*>(ws);
    float* daend = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                            align_up((size_t)p.nb * p.nch * p.H * p.P * p.N * 4, 256));
    const int npass = (p.Q * p.M + ly.R - 1) / ly.R;
    const bool wide = (int64_t)p.H * p.nch * p.nb >= kGenericStateWide;
    const int opt = wide ? 32 : 4, nslice = (p.P * p.N + 256 * opt - 1) / (256 * opt);
    MAMBA_CHECK_ARG((int64_t)p.nch * npass < 65536 && (int64_t)p.nch * nslice < 65536,
                    "too many chunks x row passes for the generic path");
    hipLaunchKernelGGL(wide ? ssd3_chunk_state_generic<32> : ssd3_chunk_state_generic<4>,
                       dim3(p.H, p.nch * nslice, p.nb), dim3(256), sm_state, stream, p, states, daend);
    MAMBA_CHECK_LAUNCH();
    hipLaunchKernelGGL(ssd3_state_pass_generic, dim3(ceil_div(p.P * p.N, 256), p.H, p.nb), dim3(256), 0, stream, p,
                       states, daend);
    MAMBA_CHECK_LAUNCH();
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    hipLaunchKernelGGL(ssd3_chunk_scan_generic, dim3(p.H, p.nch * npass, p.nb), dim3(256), sm_scan, stream, p,
                       states, ly);
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    return MAMBA_OK;
}

// The double-SSD seam's arguments as single-SSD arguments with unit coefficients.
static mamba_ssd3_args ssd3_from_double(const mamba_ssd3_double_args* d) {
    mamba_ssd3_args a{};
    a.batch = d->batch; a.seqlen = d->seqlen; a.mimo = d->mimo; a.nheads = d->nheads; a.headdim = d->headdim;
    a.ngroups = d->ngroups; a.dstate = d->dstate; a.chunk_len = d->chunk_len; a.io_dtype = d->io_dtype;
    a.v = d->v; a.v_sb = d->v_sb; a.v_sl = d->v_sl; a.v_sm = d->v_sm; a.v_sh = d->v_sh;
    a.da = d->da; a.da_sb = d->da_sb; a.da_sl = d->da_sl; a.da_sh = d->da_sh;
    a.gamma = nullptr; a.scale = nullptr;
    a.B = d->B; a.B_sb = d->B_sb; a.B_sl = d->B_sl; a.B_sm = d->B_sm; a.B_sg = d->B_sg;
    a.C = d->C; a.C_sb = d->C_sb; a.C_sl = d->C_sl; a.C_sm = d->C_sm; a.C_sg = d->C_sg;
    a.initial_state = d->initial_state;
    a.y = d->y; a.y_sb = d->y_sb; a.y_sl = d->y_sl; a.y_sm = d->y_sm; a.y_sh = d->y_sh;
    a.final_state = d->final_state;
    return a;
}

}  // namespace mamba

using namespace mamba;

extern "C" size_t mamba_ssd3_workspace_size(const mamba_ssd3_args* a) {
    Ssd3Params p;
    if (ssd3_make_params(a, &p) != MAMBA_OK) return 0;
    return ssd3_ws_bytes(p);  // the MFMA path needs none; this covers both paths
}

extern "C" int mamba_ssd3_fast_path(const mamba_ssd3_args* a) {
    Ssd3Params p;
    if (ssd3_make_params(a, &p) != MAMBA_OK) return -1;
    return ssd3_mfma_supported(a) ? 1 : 0;
}

extern "C" int mamba_ssd3_fwd(const mamba_ssd3_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream) {
    return ssd3_dispatch(a, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr, true);
}

extern "C" int mamba_ssd3_fwd_generic(const mamba_ssd3_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream) {
    return ssd3_dispatch(a, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr, false);
}

extern "C" int mamba_ssd3_fwd_timed(const mamba_ssd3_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream,
                                    void* ev_start, void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba_ssd3_fwd_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return ssd3_dispatch(a, ws, ws_bytes, (hipStream_t)stream, (hipEvent_t)ev_start, (hipEvent_t)ev_stop, true);
}

extern "C" size_t mamba_ssd3_double_workspace_size(const mamba_ssd3_double_args* d) {
    if (d == nullptr) return 0;
    const mamba_ssd3_args a = ssd3_from_double(d);
    Ssd3Params p;
    if (ssd3_make_params(&a, &p, true) != MAMBA_OK) return 0;
    return ssd3_ws_bytes(p);
}

extern "C" int mamba_ssd3_double_fast_path(const mamba_ssd3_double_args* d) {
    if (d == nullptr) return -1;
    const mamba_ssd3_args a = ssd3_from_double(d);
    Ssd3Params p;
    if (ssd3_make_params(&a, &p, true) != MAMBA_OK) return -1;
    return ssd3_mfma_supported(&a) ? 1 : 0;
}

extern "C" int mamba_ssd3_double_fwd(const mamba_ssd3_double_args* d, void* ws, size_t ws_bytes,
                                     mamba_stream_t stream) {
    if (d == nullptr) {
        set_error("args is NULL");
        return MAMBA_ERR_INVALID_ARG;
    }
    const mamba_ssd3_args a = ssd3_from_double(d);
    return ssd3_dispatch(&a, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr, true, true);
}

extern "C" int mamba_ssd3_double_fwd_generic(const mamba_ssd3_double_args* d, void* ws, size_t ws_bytes,
                                             mamba_stream_t stream) {
    if (d == nullptr) {
        set_error("args is NULL");
        return MAMBA_ERR_INVALID_ARG;
    }
    const mamba_ssd3_args a = ssd3_from_double(d);
    return ssd3_dispatch(&a, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr, false, true);
}
