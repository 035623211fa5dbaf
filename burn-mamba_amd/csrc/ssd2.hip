// Mamba-2 chunked SSD forward for gfx950.
//
// Two code paths behind one entry point (mamba_ssd2_fwd):
//   * the MFMA path (ssd2_mfma.hip) for bf16 I/O, headdim 64, dstate 64/128
//     and chunk lengths that are multiples of 32 up to 256;
//   * the shape-generic path below for everything else: three SIMT kernels
//     (chunk state, state passing, chunk scan) with f32 arithmetic.
//
// Reference: src/mamba2/ssd/serial.rs:34-506 (K1..K5) and the trait default
// body src/mamba2/ssd/serial_recalculated/serial_recalculated.rs:98-155.

#include "common.h"
#include "ssd2.h"

namespace mamba {

// ------------------------------------------------------------ block scan --
// Inclusive prefix sum of one value per thread over a 256-thread block.
__device__ __forceinline__ float block_incl_scan256(float v, float* sh4) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_incl_scan(v);
    if (lane == 63) sh4[wid] = v;
    __syncthreads();
    float off = 0.f;
    for (int w = 0; w < wid; ++w) off += sh4[w];
    __syncthreads();
    return v + off;
}

// Fills cs[0..Q) with the intra-chunk cumulative sum of dt*A (K1,
// serial.rs:138-164) and dts[0..Q) with dt; positions past seqlen read as
// dt = 0, which is exactly the zero padding of mamba2.rs:709-722.
__device__ void chunk_cumsum(const Ssd2Params& p, int b, int c, int h, float* cs, float* dts,
                             float* sh4) {
    const float a = p.A[h];
    float carry = 0.f;
    for (int base = 0; base < p.Q; base += 256) {
        const int l = base + threadIdx.x;
        const int t = c * p.Q + l;
        float dtv = 0.f;
        if (l < p.Q && t < p.L) dtv = p.dt[(int64_t)b * p.dt_sb + (int64_t)t * p.dt_sl + (int64_t)h * p.dt_sh];
        float s = block_incl_scan256(dtv * a, sh4) + carry;
        if (l < p.Q) {
            cs[l] = s;
            dts[l] = dtv;
        }
        // carry = last element of this 256-segment
        __syncthreads();
        const int last = min(base + 256, p.Q) - 1;
        carry = cs[last];
        __syncthreads();
    }
}

// ------------------------------------------------------- K1 + K3 (generic) --
// S[b,c,h,p,n] = sum_l x[l,p] * (B[l,n] * (exp(cs_end - cs_l) * dt_l))
// One workgroup per (head, chunk x slice of 256 OPT entries, batch), OPT
// entries per thread: the launch takes OPT = 4 when (head, chunk, batch) alone
// would give few workgroups (short sequences), else 32 (each slice stages the
// chunk's x and weighted B rows once, so fewer slices stage less).
template <typename T, int OPT>
__global__ __launch_bounds__(256) void ssd2_chunk_state_generic(Ssd2Params p, float* states,
                                                                float* da_end) {
    extern __shared__ float smem[];
    const int nslice = (p.P * p.N + 256 * OPT - 1) / (256 * OPT);
    const int h = blockIdx.x, c = blockIdx.y / nslice, slice = blockIdx.y % nslice, b = blockIdx.z;
    const int g = h / (p.H / p.G);
    const int Q = p.Q, P = p.P, N = p.N;
    float* cs = smem;            // [Q]
    float* dts = cs + Q;         // [Q]
    float* sh4 = dts + Q;        // [4]
    float* xt = sh4 + 4;         // [TL][P]
    constexpr int TL = 16;
    float* bt = xt + TL * P;     // [TL][N]
    chunk_cumsum(p, b, c, h, cs, dts, sh4);
    const float cs_end = cs[Q - 1];
    if (threadIdx.x == 0 && slice == 0) da_end[((int64_t)b * p.H + h) * p.nch + c] = cs_end;
    const T* X = (const T*)p.x;
    const T* Bm = (const T*)p.Bm;
    float* Sout = states + (((int64_t)b * p.nch + c) * p.H + h) * P * N;
    {
        const int e0 = slice * 256 * OPT;
        float acc[OPT];
#pragma unroll
        for (int k = 0; k < OPT; ++k) acc[k] = 0.f;
        for (int l0 = 0; l0 < Q; l0 += TL) {
            __syncthreads();
            for (int i = threadIdx.x; i < TL * P; i += 256) {
                const int l = l0 + i / P, pp = i % P, t = c * Q + l;
                xt[i] = (l < Q && t < p.L)
                            ? load_f32(X + (int64_t)b * p.x_sb + (int64_t)t * p.x_sl + (int64_t)h * p.x_sh + pp)
                            : 0.f;
            }
            for (int i = threadIdx.x; i < TL * N; i += 256) {
                const int l = l0 + i / N, n = i % N, t = c * Q + l;
                float w = 0.f;
                if (l < Q && t < p.L) {
                    const float scale = expf(cs_end - cs[l]) * dts[l];
                    w = load_f32(Bm + (int64_t)b * p.B_sb + (int64_t)t * p.B_sl + (int64_t)g * p.B_sg + n) * scale;
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
                    for (int l = 0; l < TL; ++l) a += xt[l * P + pp] * bt[l * N + n];
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

// ------------------------------------------------------------ K4 (generic) --
// In place: states[c] <- state entering chunk c; final <- state after the last.
__global__ __launch_bounds__(256) void ssd2_state_pass_generic(Ssd2Params p, float* states,
                                                               const float* da_end) {
    const int h = blockIdx.y, b = blockIdx.z;
    const int PN = p.P * p.N;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= PN) return;
    float run = p.h0 ? p.h0[((int64_t)b * p.H + h) * PN + e] : 0.f;
    if (p.init_hpr) run += p.init_hpr[(int64_t)h * PN + e];
    const float* de = da_end + ((int64_t)b * p.H + h) * p.nch;
    for (int c = 0; c < p.nch; ++c) {
        float* s = states + (((int64_t)b * p.nch + c) * p.H + h) * PN + e;
        const float tmp = *s;
        *s = run;
        run = expf(de[c]) * run + tmp;
    }
    p.hT[((int64_t)b * p.H + h) * PN + e] = run;
}

// ------------------------------------------------------- K2 + K5 (generic) --
// One workgroup per (head, chunk x pass of R rows, batch):
//   y[i][p] = exp(cs_i) C_i.h_in[p] + sum_{j <= i} W[i][j] x[j][p] + D x[i][p],
//   W[i][j] = (C_i.B_j) exp(cs_i - cs_j) dt_j  (serial.rs:170-230, K2 + K5).
// The pass forms its rows of W in LDS once per (row, source), its B rows
// staged 32 at a time (padded rows: consecutive sources on different banks);
// then thread (column p, row slot rs) accumulates RR rows of one column, each
// x load serving all of them.
struct Ssd2ScanLds {
    int R, RR, TP;  // rows per pass, rows per thread, row slots (256 / P)
    bool h_lds;     // h_in staged in LDS
};
constexpr int kSsd2BT = 32;

template <typename T>
__global__ __launch_bounds__(256) void ssd2_chunk_scan_generic(Ssd2Params p, const float* states, Ssd2ScanLds ly) {
    extern __shared__ float smem[];
    const int npass = (p.Q + ly.R - 1) / ly.R;
    const int h = blockIdx.x, c = blockIdx.y / npass, pass = blockIdx.y % npass, b = blockIdx.z;
    const int g = h / (p.H / p.G);
    const int Q = p.Q, P = p.P, N = p.N, R = ly.R, RR = ly.RR, TP = ly.TP, NB = N + 1;
    float* cs = smem;            // [Q]
    float* dts = cs + Q;         // [Q]
    float* sh4 = dts + Q;        // [4]
    float* W = sh4 + 4;          // [R][Q]
    float* Cs = W + R * Q;       // [R][N]
    float* Bt = Cs + R * N;      // [kSsd2BT][NB]
    float* Hs = Bt + kSsd2BT * NB;  // [N][P] (h_lds)
    chunk_cumsum(p, b, c, h, cs, dts, sh4);
    const T* X = (const T*)p.x;
    const T* Bm = (const T*)p.Bm;
    const T* Cm = (const T*)p.Cm;
    T* Y = (T*)p.y;
    const float* hin = states + (((int64_t)b * p.nch + c) * p.H + h) * P * N;
    const float Dh = p.D ? p.D[h] : 0.f;
    const int qvalid = min(Q, p.L - c * Q);
    const int i0 = pass * R;
    if (i0 >= qvalid) return;  // a pass past the last chunk's end (workgroup-uniform)
    if (ly.h_lds)
        for (int k = threadIdx.x; k < P * N; k += 256) Hs[(k % N) * P + k / N] = hin[k];
    for (int k = threadIdx.x; k < R * N; k += 256) {
        const int ii = i0 + k / N;
        Cs[k] = ii < qvalid ? load_f32(Cm + (int64_t)b * p.C_sb + (int64_t)(c * Q + ii) * p.C_sl + (int64_t)g * p.C_sg + k % N)
                            : 0.f;
    }
    __syncthreads();
    const int nsrc = min(i0 + R, qvalid);  // sources up to the pass's last row
    for (int s0 = 0; s0 < nsrc; s0 += kSsd2BT) {
        for (int k = threadIdx.x; k < kSsd2BT * N; k += 256) {
            const int jj = k / N, j = s0 + jj;
            Bt[jj * NB + k % N] =
                j < nsrc ? load_f32(Bm + (int64_t)b * p.B_sb + (int64_t)(c * Q + j) * p.B_sl + (int64_t)g * p.B_sg + k % N)
                         : 0.f;
        }
        __syncthreads();
        for (int k = threadIdx.x; k < R * kSsd2BT; k += 256) {
            const int r = k / kSsd2BT, jj = k % kSsd2BT, j = s0 + jj, ii = i0 + r;
            if (j >= nsrc) continue;
            float v = 0.f;
            if (ii < qvalid && j <= ii) {
                const float* cr = Cs + r * N;
                const float* br = Bt + jj * NB;
                float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
                int n = 0;
                for (; n + 4 <= N; n += 4) {
                    d0 = __builtin_fmaf(cr[n], br[n], d0);
                    d1 = __builtin_fmaf(cr[n + 1], br[n + 1], d1);
                    d2 = __builtin_fmaf(cr[n + 2], br[n + 2], d2);
                    d3 = __builtin_fmaf(cr[n + 3], br[n + 3], d3);
                }
                for (; n < N; ++n) d0 = __builtin_fmaf(cr[n], br[n], d0);
                v = ((d0 + d1) + (d2 + d3)) * expf(cs[ii] - cs[j]) * dts[j];
            }
            W[r * Q + j] = v;
        }
        __syncthreads();
    }
    const int pp = threadIdx.x % P, rs = threadIdx.x / P;
    if (rs >= TP) return;
    float acc[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] = 0.f;
    constexpr int U = 16;  // sources whose x loads are issued together
    for (int j0 = 0; j0 < nsrc; j0 += U) {
        float xv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + u, nsrc - 1);  // clamped: its W entries below are skipped
            xv[u] = load_f32(X + (int64_t)b * p.x_sb + (int64_t)(c * Q + j) * p.x_sl + (int64_t)h * p.x_sh + pp);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (j0 + u >= nsrc) break;
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (k < RR) acc[k] = __builtin_fmaf(W[(rs + TP * k) * Q + j0 + u], xv[u], acc[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        if (k >= RR) break;
        const int r = rs + TP * k, ii = i0 + r;
        if (ii >= qvalid) continue;
        const int ti = c * Q + ii;
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
        const float xi = load_f32(X + (int64_t)b * p.x_sb + (int64_t)ti * p.x_sl + (int64_t)h * p.x_sh + pp);
        store_f32(Y + (int64_t)b * p.y_sb + (int64_t)ti * p.y_sl + (int64_t)h * p.y_sh + pp,
                  __builtin_fmaf((b0 + b1), expf(cs[ii]), acc[k]) + Dh * xi);
    }
}

// The chunk scan's pass geometry and its dynamic LDS bytes (0: does not fit).
static size_t ssd2_scan_layout(const Ssd2Params& p, Ssd2ScanLds* ly) {
    const int TP = p.P >= 256 ? 1 : 256 / p.P;
    const size_t limit = 64 * 1024 / 4;  // words
    const size_t fixed = 2 * (size_t)p.Q + 4 + (size_t)kSsd2BT * (p.N + 1);
    int RR = TP >= 16 ? 1 : 16 / TP;
    while (RR > 1 && fixed + (size_t)TP * RR * ((size_t)p.Q + p.N) > limit) RR /= 2;
    ly->TP = TP; ly->RR = RR; ly->R = TP * RR;
    size_t words = fixed + (size_t)ly->R * ((size_t)p.Q + p.N);
    if (words > limit) return 0;
    ly->h_lds = words + (size_t)p.P * p.N <= limit;
    if (ly->h_lds) words += (size_t)p.P * p.N;
    return words * 4;
}

// ------------------------------------------------------------ host side --
size_t ssd2_generic_workspace(const Ssd2Params& p) {
    const size_t states = (size_t)p.nb * p.nch * p.H * p.P * p.N * sizeof(float);
    const size_t daend = (size_t)p.nb * p.H * p.nch * sizeof(float);
    return align_up(states, 256) + align_up(daend, 256);
}

int ssd2_generic_launch(const Ssd2Params& p, void* ws, hipStream_t stream, hipEvent_t ev0,
                        hipEvent_t ev1) {
    float* states = (float*)ws;
    float* daend = (float*)((char*)ws + align_up((size_t)p.nb * p.nch * p.H * p.P * p.N * sizeof(float), 256));
    dim3 grid(p.H, p.nch, p.nb);
    const size_t sm_state = (2 * (size_t)p.Q + 4 + 16 * (size_t)p.P + 16 * (size_t)p.N) * sizeof(float);
    Ssd2ScanLds ly;
    const size_t sm_scan = ssd2_scan_layout(p, &ly);
    const int npass = (p.Q + ly.R - 1) / ly.R;
    MAMBA_CHECK_ARG(sm_scan > 0 && (int64_t)p.nch * npass < 65536, "chunk too large for the generic path");
    const dim3 gscan(p.H, p.nch * npass, p.nb);
    const bool wide = (int64_t)p.H * p.nch * p.nb >= kGenericStateWide;
    const int opt = wide ? 32 : 4, nslice = (p.P * p.N + 256 * opt - 1) / (256 * opt);
    MAMBA_CHECK_ARG((int64_t)p.nch * nslice < 65536, "too many chunks for the generic path");
    const dim3 gstate(p.H, p.nch * nslice, p.nb);
    const bool bf = p.io_dtype == MAMBA_BF16;
    auto state_kernel = wide ? (bf ? ssd2_chunk_state_generic<bf16_t, 32> : ssd2_chunk_state_generic<float, 32>)
                             : (bf ? ssd2_chunk_state_generic<bf16_t, 4> : ssd2_chunk_state_generic<float, 4>);
    hipLaunchKernelGGL(state_kernel, gstate, dim3(256), sm_state, stream, p, states, daend);
    MAMBA_CHECK_LAUNCH();
    dim3 gpass(ceil_div(p.P * p.N, 256), p.H, p.nb);
    hipLaunchKernelGGL(ssd2_state_pass_generic, gpass, dim3(256), 0, stream, p, states, daend);
    MAMBA_CHECK_LAUNCH();
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    if (p.io_dtype == MAMBA_BF16) {
        hipLaunchKernelGGL(ssd2_chunk_scan_generic<bf16_t>, gscan, dim3(256), sm_scan, stream, p, states, ly);
    } else {
        hipLaunchKernelGGL(ssd2_chunk_scan_generic<float>, gscan, dim3(256), sm_scan, stream, p, states, ly);
    }
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    return MAMBA_OK;
}

// Host-side validation of the public arguments (the reference asserts the same
// conditions: mamba2.rs:562-566, serial_recalculated.rs:41-44, gqa.rs:37-41).
int ssd2_make_params(const mamba_ssd2_args* a, Ssd2Params* out) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0, "batch and seqlen must be >= 1");
    MAMBA_CHECK_ARG(a->nheads > 0 && a->headdim > 0 && a->dstate > 0, "nheads/headdim/dstate must be >= 1");
    MAMBA_CHECK_ARG(a->ngroups > 0 && a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    MAMBA_CHECK_ARG(a->chunk_len > 0 && a->chunk_len <= 1024, "chunk_len must be in [1, 1024]");
    MAMBA_CHECK_ARG(a->io_dtype == MAMBA_F32 || a->io_dtype == MAMBA_BF16, "io_dtype must be MAMBA_F32 or MAMBA_BF16");
    MAMBA_CHECK_ARG(a->x && a->dt && a->A && a->B && a->C && a->y && a->final_state,
                    "x, dt, A, B, C, y and final_state are required");
    MAMBA_CHECK_ARG(a->headdim <= 256 && a->dstate <= 256, "headdim and dstate must be <= 256");
    Ssd2Params& p = *out;
    p.nb = a->batch; p.L = a->seqlen; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups;
    p.N = a->dstate; p.Q = a->chunk_len; p.nch = (a->seqlen + a->chunk_len - 1) / a->chunk_len;
    p.io_dtype = a->io_dtype;
    p.x = a->x; p.x_sb = a->x_sb; p.x_sl = a->x_sl; p.x_sh = a->x_sh;
    p.dt = a->dt; p.dt_sb = a->dt_sb; p.dt_sl = a->dt_sl; p.dt_sh = a->dt_sh;
    p.A = a->A; p.D = a->D;
    p.Bm = a->B; p.B_sb = a->B_sb; p.B_sl = a->B_sl; p.B_sg = a->B_sg;
    p.Cm = a->C; p.C_sb = a->C_sb; p.C_sl = a->C_sl; p.C_sg = a->C_sg;
    p.h0 = a->initial_state; p.init_hpr = a->init_state_hpr;
    p.y = a->y; p.y_sb = a->y_sb; p.y_sl = a->y_sl; p.y_sh = a->y_sh;
    p.hT = a->final_state;
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" size_t mamba_ssd2_workspace_size(const mamba_ssd2_args* a) {
    Ssd2Params p;
    if (ssd2_make_params(a, &p) != MAMBA_OK) return 0;
    size_t ws = ssd2_generic_workspace(p);
    const size_t fast = ssd2_mfma_workspace(p);
    return ws > fast ? ws : fast;
}

extern "C" int mamba_ssd2_fast_path(const mamba_ssd2_args* a) {
    Ssd2Params p;
    if (ssd2_make_params(a, &p) != MAMBA_OK) return -1;
    return ssd2_mfma_supported(p) ? 1 : 0;
}

extern "C" int mamba_ssd2_fwd_generic(const mamba_ssd2_args* a, void* ws, size_t ws_bytes,
                                      mamba_stream_t stream) {
    Ssd2Params p;
    int st = ssd2_make_params(a, &p);
    if (st != MAMBA_OK) return st;
    if (ws == nullptr || ws_bytes < ssd2_generic_workspace(p)) {
        set_error("mamba_ssd2_fwd_generic: workspace missing or too small");
        return MAMBA_ERR_WORKSPACE;
    }
    return ssd2_generic_launch(p, ws, (hipStream_t)stream);
}

static int ssd2_dispatch(const mamba_ssd2_args* a, void* ws, size_t ws_bytes, hipStream_t stream,
                         hipEvent_t ev0, hipEvent_t ev1) {
    Ssd2Params p;
    int st = ssd2_make_params(a, &p);
    if (st != MAMBA_OK) return st;
    if (ssd2_mfma_supported(p)) {
        if (ws == nullptr || ws_bytes < ssd2_mfma_workspace(p)) {
            set_error("mamba_ssd2_fwd: workspace missing or too small");
            return MAMBA_ERR_WORKSPACE;
        }
        return ssd2_mfma_launch(p, ws, stream, ev0, ev1);
    }
    if (ws == nullptr || ws_bytes < ssd2_generic_workspace(p)) {
        set_error("mamba_ssd2_fwd: workspace missing or too small");
        return MAMBA_ERR_WORKSPACE;
    }
    return ssd2_generic_launch(p, ws, stream, ev0, ev1);
}

extern "C" int mamba_ssd2_fwd(const mamba_ssd2_args* a, void* ws, size_t ws_bytes,
                              mamba_stream_t stream) {
    return ssd2_dispatch(a, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba_ssd2_fwd_timed(const mamba_ssd2_args* a, void* ws, size_t ws_bytes,
                                    mamba_stream_t stream, void* ev_start, void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba_ssd2_fwd_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return ssd2_dispatch(a, ws, ws_bytes, (hipStream_t)stream, (hipEvent_t)ev_start,
                         (hipEvent_t)ev_stop);
}
