// Mamba-1 selective scan for gfx950 (f32).
//
// Reference: Mamba1::selective_scan (src/mamba1/mamba1.rs:422-523), the
// optional dt_proj bias + softplus of Mamba1::ssm (mamba1.rs:391-394) and the
// silu(z) gate of Mamba1::forward (mamba1.rs:348):
//   a = exp(delta_t A[d, n]);  h_n <- a h_n + delta_t B_n(t) u_t
//   y_t = (sum_n C_n(t) h_n + D u_t) * silu(z_t)
//
// There is no matrix product here: every (channel, state) pair has its own
// decay, so the work is VALU-bound (one exp, two multiplies and two FMAs per
// state per token).  A workgroup owns 64 channels of one batch row; each
// channel is spread over N/4 lanes holding 4 states each, so for dstate 16 the
// per-token y reduction is a quad DPP sum.  Time is processed in tiles of 16 tokens that
// are staged through LDS with coalesced loads (the next tile's loads are issued
// into registers before the current tile is computed); softplus, delta*u, D*u
// and silu(z) are evaluated once per element in the staging pass.

#include <cstdlib>

#include "common.h"

namespace mamba {

struct Mamba1Params {
    int nb, D, L, N;
    const float* u; int64_t u_sb, u_sd, u_sl;
    const float* dl; int64_t dl_sb, dl_sd, dl_sl;
    const float* A; int64_t A_sd, A_sn;
    const float* Bm; int64_t B_sb, B_sn, B_sl;
    const float* Cm; int64_t C_sb, C_sn, C_sl;
    const float* Dv; const float* z; int64_t z_sb, z_sd, z_sl;
    const float* dbias; int softplus;
    const float* h0;
    float* y; int64_t y_sb, y_sd, y_sl;
    float* hT;
};

constexpr float kLog2eM1 = 1.4426950408889634f;
constexpr int kTT = 16;  // tokens per staged tile (32 measured slower: the staging registers spill)

// softplus(x) = log(1 + e^x); above 20 it equals x to f32 precision (the
// reference's Burn softplus overflows to inf above ~88.7 instead).
__device__ __forceinline__ float m1_softplus(float x) {
    return x > 20.f ? x : log1pf(__expf(x));
}

__device__ __forceinline__ float quad_sum(float v) {
    // xor 1 then xor 2 inside each quad of lanes (DPP quad_perm)
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    return v;
}

// NS = lanes per channel (N / 4); a workgroup holds CPB = 64 channels, i.e.
// 16 N threads (256 for the common dstate 16).
template <int N, bool TM>
__global__ __launch_bounds__(16 * N, N <= 16 ? 3 : 1) void mamba1_scan_kernel(Mamba1Params p) {
    constexpr int NS = N / 4;
    constexpr int CPB = 64;
    constexpr int NT = CPB * NS;                  // threads per workgroup
    constexpr int TP = kTT + 1;  // LDS row pitch (floats)
    constexpr int EPT = CPB * kTT / NT;           // per-channel elements per thread per tile
    constexpr int BPT = (N * kTT + NT - 1) / NT;  // B/C elements per thread per tile
    __shared__ float2 s_ddu[CPB][TP];  // (delta, delta * u)
    __shared__ float2 s_epi[CPB][TP];  // (D * u, silu(z))
    __shared__ float s_y[CPB][TP];
    __shared__ __align__(16) float s_B[kTT][N];
    __shared__ __align__(16) float s_C[kTT][N];

    const int tid = threadIdx.x;
    const int nblk_d = (p.D + CPB - 1) / CPB;
    const int b = blockIdx.x / nblk_d, d0 = (blockIdx.x % nblk_d) * CPB;
    // compute mapping: channel c of this block, states 4*ng .. 4*ng+3
    const int c = tid / NS, ng = tid % NS;
    const int d = d0 + c;
    const bool dvalid = d < p.D;
    float A2[4], h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int n = 4 * ng + k;
        A2[k] = dvalid ? p.A[(int64_t)d * p.A_sd + (int64_t)n * p.A_sn] * kLog2eM1 : 0.f;
        h[k] = (dvalid && p.h0) ? p.h0[((int64_t)b * p.D + d) * N + n] : 0.f;
    }
    // load mapping: element e of this thread -> (channel lc, token lt) of the
    // tile, read along time when the inputs are time-contiguous (TM) and along
    // channels otherwise.  u, delta, z and y share one stride pair (checked on
    // the host), so one loop-invariant 32-bit offset addresses all four.
    // NT is a multiple of kTT and of CPB, so element e of a thread sits a
    // fixed step from its element 0: e_off(e) = e_base + e * e_step.
    static_assert(NT % kTT == 0 && NT % CPB == 0, "element steps must be uniform");
    auto e_lc = [&](int e) { return TM ? tid / kTT + (NT / kTT) * e : tid % CPB; };
    auto e_lt = [&](int e) { return TM ? tid % kTT : tid / CPB + (NT / CPB) * e; };
    const int e_base = (int)((int64_t)(d0 + e_lc(0)) * p.u_sd + (int64_t)e_lt(0) * p.u_sl);
    const int e_step = (int)(TM ? (int64_t)(NT / kTT) * p.u_sd : (int64_t)(NT / CPB) * p.u_sl);
    auto e_off = [&](int e) { return e_base + e * e_step; };
    const float* ub = p.u + (int64_t)b * p.u_sb;
    const float* db = p.dl + (int64_t)b * p.dl_sb;
    const float* zb = p.z ? p.z + (int64_t)b * p.z_sb : nullptr;
    float* yb = p.y + (int64_t)b * p.y_sb;
    const float* Bb = p.Bm + (int64_t)b * p.B_sb;
    const float* Cb = p.Cm + (int64_t)b * p.C_sb;
    float ru[EPT], rd[EPT], rz[EPT], rB[BPT], rC[BPT];
    auto fetch = [&](int t0) {
        const int64_t tb = (int64_t)t0 * p.u_sl;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const bool ok = d0 + e_lc(e) < p.D && t0 + e_lt(e) < p.L;
            ru[e] = ok ? ub[tb + e_off(e)] : 0.f;
            rd[e] = ok ? db[tb + e_off(e)] : 0.f;
            rz[e] = (ok && zb) ? zb[tb + e_off(e)] : 0.f;
        }
#pragma unroll
        for (int e = 0; e < BPT; ++e) {
            const int idx = tid + NT * e;
            const int n = idx % N, lt = idx / N, t = t0 + lt;
            const bool ok = idx < N * kTT && t < p.L;
            rB[e] = ok ? Bb[(int64_t)n * p.B_sn + (int64_t)t * p.B_sl] : 0.f;
            rC[e] = ok ? Cb[(int64_t)n * p.C_sn + (int64_t)t * p.C_sl] : 0.f;
        }
    };
    fetch(0);
    const int ntile = (p.L + kTT - 1) / kTT;
    for (int tile = 0; tile < ntile; ++tile) {
        const int t0 = tile * kTT;
        // ---- stage: per-element preprocessing into LDS
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const int lc = e_lc(e), lt = e_lt(e);
            const int dd = d0 + lc;
            float dv = rd[e];
            if (p.dbias && dd < p.D) dv += p.dbias[dd];
            if (p.softplus) dv = m1_softplus(dv);
            if (t0 + lt >= p.L) dv = 0.f;  // past the end: identity step, y unused
            const float Dd = (p.Dv && dd < p.D) ? p.Dv[dd] : 0.f;
            const float g = p.z ? rz[e] * __builtin_amdgcn_rcpf(1.f + __expf(-rz[e])) : 1.f;
            s_ddu[lc][lt] = make_float2(dv, dv * ru[e]);
            s_epi[lc][lt] = make_float2(Dd * ru[e], g);
        }
#pragma unroll
        for (int e = 0; e < BPT; ++e) {
            const int idx = tid + NT * e;
            if (idx < N * kTT) {
                s_B[idx / N][idx % N] = rB[e];
                s_C[idx / N][idx % N] = rC[e];
            }
        }
        __syncthreads();
        if (tile + 1 < ntile) fetch(t0 + kTT);
        // ---- recurrence over the tile's tokens, in groups of 4: the LDS reads
        // of a group are issued together and its 4 quad reductions are
        // independent, so neither the LDS latency nor the DPP hazards serialise
#pragma unroll 1
        for (int lt0 = 0; lt0 < kTT; lt0 += 4) {
            float2 dd[4];
            float4 bq[4], cq[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                dd[g] = s_ddu[c][lt0 + g];
                bq[g] = *(const float4*)&s_B[lt0 + g][4 * ng];
                cq[g] = *(const float4*)&s_C[lt0 + g][4 * ng];
            }
            float yq[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float a0 = __builtin_amdgcn_exp2f(dd[g].x * A2[0]);
                const float a1 = __builtin_amdgcn_exp2f(dd[g].x * A2[1]);
                const float a2 = __builtin_amdgcn_exp2f(dd[g].x * A2[2]);
                const float a3 = __builtin_amdgcn_exp2f(dd[g].x * A2[3]);
                h[0] = __builtin_fmaf(h[0], a0, dd[g].y * bq[g].x);
                h[1] = __builtin_fmaf(h[1], a1, dd[g].y * bq[g].y);
                h[2] = __builtin_fmaf(h[2], a2, dd[g].y * bq[g].z);
                h[3] = __builtin_fmaf(h[3], a3, dd[g].y * bq[g].w);
                yq[g] = __builtin_fmaf(cq[g].x, h[0], cq[g].y * h[1]) +
                        __builtin_fmaf(cq[g].z, h[2], cq[g].w * h[3]);
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if constexpr (NS == 4) {
                    yq[g] = quad_sum(yq[g]);
                } else {
#pragma unroll
                    for (int o = 1; o < NS; o <<= 1) yq[g] += __shfl_xor(yq[g], o, 64);
                }
            }
            // every lane of the channel holds the sum; one store per channel
            // lane group is enough, but a uniform store avoids exec toggling
#pragma unroll
            for (int g = 0; g < 4; ++g) s_y[c][lt0 + g] = yq[g];
        }
        __syncthreads();  // s_y complete before the epilogue reads it
        // ---- epilogue + store: y = (sum_n C h + D u) * silu(z)
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const int lc = e_lc(e), lt = e_lt(e);
            if (d0 + lc < p.D && t0 + lt < p.L) {
                const float2 ep = s_epi[lc][lt];
                yb[(int64_t)t0 * p.u_sl + e_off(e)] = (s_y[lc][lt] + ep.x) * ep.y;
            }
        }
        __syncthreads();
    }
    if (dvalid && p.hT) {
#pragma unroll
        for (int k = 0; k < 4; ++k) p.hT[((int64_t)b * p.D + d) * N + 4 * ng + k] = h[k];
    }
}

// Shape-generic fallback (any dstate <= 256): one thread per channel, states in
// LDS.  Used when dstate is not 16, 32 or 64 or the strides do not allow the
// tiled kernel.
__global__ __launch_bounds__(64) void mamba1_scan_generic(Mamba1Params p) {
    extern __shared__ float s_h[];  // [64][N]
    const int ch = blockIdx.x * 64 + threadIdx.x;
    if (ch >= p.nb * p.D) return;
    const int b = ch / p.D, d = ch % p.D;
    float* h = s_h + threadIdx.x * p.N;
    for (int n = 0; n < p.N; ++n) h[n] = p.h0 ? p.h0[(int64_t)ch * p.N + n] : 0.f;
    const float Dd = p.Dv ? p.Dv[d] : 0.f;
    for (int t = 0; t < p.L; ++t) {
        float dv = p.dl[(int64_t)b * p.dl_sb + (int64_t)d * p.dl_sd + (int64_t)t * p.dl_sl];
        if (p.dbias) dv += p.dbias[d];
        if (p.softplus) dv = m1_softplus(dv);
        const float uv = p.u[(int64_t)b * p.u_sb + (int64_t)d * p.u_sd + (int64_t)t * p.u_sl];
        float acc = 0.f;
        for (int n = 0; n < p.N; ++n) {
            const float a = __expf(dv * p.A[(int64_t)d * p.A_sd + (int64_t)n * p.A_sn]);
            const float bv = p.Bm[(int64_t)b * p.B_sb + (int64_t)n * p.B_sn + (int64_t)t * p.B_sl];
            const float cv = p.Cm[(int64_t)b * p.C_sb + (int64_t)n * p.C_sn + (int64_t)t * p.C_sl];
            h[n] = h[n] * a + (dv * bv) * uv;
            acc += h[n] * cv;
        }
        float out = acc + Dd * uv;
        if (p.z) {
            const float zv = p.z[(int64_t)b * p.z_sb + (int64_t)d * p.z_sd + (int64_t)t * p.z_sl];
            out *= zv / (1.f + __expf(-zv));
        }
        p.y[(int64_t)b * p.y_sb + (int64_t)d * p.y_sd + (int64_t)t * p.y_sl] = out;
    }
    if (p.hT)
        for (int n = 0; n < p.N; ++n) p.hT[(int64_t)ch * p.N + n] = h[n];
}

static int m1_make_params(const mamba1_scan_args* a, Mamba1Params* out) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->dim > 0 && a->seqlen > 0, "batch, dim and seqlen must be >= 1");
    MAMBA_CHECK_ARG(a->dstate > 0 && a->dstate <= 256, "dstate must be in [1, 256]");
    MAMBA_CHECK_ARG(a->u && a->delta && a->A && a->B && a->C && a->y, "u, delta, A, B, C and y are required");
    Mamba1Params& p = *out;
    p.nb = a->batch; p.D = a->dim; p.L = a->seqlen; p.N = a->dstate;
    p.u = a->u; p.u_sb = a->u_sb; p.u_sd = a->u_sd; p.u_sl = a->u_sl;
    p.dl = a->delta; p.dl_sb = a->delta_sb; p.dl_sd = a->delta_sd; p.dl_sl = a->delta_sl;
    p.A = a->A; p.A_sd = a->A_sd; p.A_sn = a->A_sn;
    p.Bm = a->B; p.B_sb = a->B_sb; p.B_sn = a->B_sn; p.B_sl = a->B_sl;
    p.Cm = a->C; p.C_sb = a->C_sb; p.C_sn = a->C_sn; p.C_sl = a->C_sl;
    p.Dv = a->D; p.z = a->z; p.z_sb = a->z_sb; p.z_sd = a->z_sd; p.z_sl = a->z_sl;
    p.dbias = a->delta_bias; p.softplus = a->delta_softplus != 0;
    p.h0 = a->initial_state;
    p.y = a->y; p.y_sb = a->y_sb; p.y_sd = a->y_sd; p.y_sl = a->y_sl;
    p.hT = a->final_state;
    return MAMBA_OK;
}

template <int N>
static void launch_m1(const Mamba1Params& p, hipStream_t stream) {
    constexpr int CPB = 64;
    const int nblk = p.nb * ((p.D + CPB - 1) / CPB);
    if (p.u_sl == 1)
        hipLaunchKernelGGL((mamba1_scan_kernel<N, true>), dim3(nblk), dim3(16 * N), 0, stream, p);
    else
        hipLaunchKernelGGL((mamba1_scan_kernel<N, false>), dim3(nblk), dim3(16 * N), 0, stream, p);
}

static int m1_dispatch(const mamba1_scan_args* a, hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    Mamba1Params p;
    int st = m1_make_params(a, &p);
    if (st != MAMBA_OK) return st;
    const bool same_strides = p.dl_sd == p.u_sd && p.dl_sl == p.u_sl && p.y_sd == p.u_sd &&
                              p.y_sl == p.u_sl && (!p.z || (p.z_sd == p.u_sd && p.z_sl == p.u_sl));
    const bool fits32 = (int64_t)p.D * std::abs(p.u_sd) + (int64_t)p.L * std::abs(p.u_sl) < (1ll << 31);
    const int nfast = (same_strides && fits32) ? p.N : 0;
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    switch (nfast) {
        case 16: launch_m1<16>(p, stream); break;
        case 32: launch_m1<32>(p, stream); break;
        case 64: launch_m1<64>(p, stream); break;
        default: {
            const int nblk = ceil_div(p.nb * p.D, 64);
            hipLaunchKernelGGL(mamba1_scan_generic, dim3(nblk), dim3(64), 64 * p.N * sizeof(float), stream, p);
        }
    }
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" int mamba1_scan_fwd(const mamba1_scan_args* a, mamba_stream_t stream) {
    return m1_dispatch(a, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba1_scan_fwd_timed(const mamba1_scan_args* a, mamba_stream_t stream, void* ev_start,
                                     void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba1_scan_fwd_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return m1_dispatch(a, (hipStream_t)stream, (hipEvent_t)ev_start, (hipEvent_t)ev_stop);
}
