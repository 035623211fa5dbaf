// Mamba-1 recurrent decode step for gfx950 (f32), and the depthwise causal
// conv-window step shared by the recurrent blocks.
//
// Reference: Mamba1::selective_scan_step (burn-mamba src/mamba1/mamba1.rs:666-733)
// with the dt_proj bias + softplus of Mamba1::ssm_step (:646) and the silu(res)
// gate of Mamba1::step (:603); the conv window roll + depthwise dot + bias +
// SiLU of Mamba1::step (:558-597).
//
// One token per sequence: the state [b, d, n] is read and written once, so the
// step is HBM-bound (8 bytes of state traffic per (channel, state) against
// ~6 flops).  For dstate a multiple of 4 (up to 64) a channel is spread over
// n/4 lanes holding 4 consecutive states each: consecutive lanes touch
// consecutive 16 bytes, and y = sum_n h C is a butterfly over those lanes.
#include "common.h"

namespace mamba {

struct M1StepParams {
    int nb, D, N;
    const float* u; int64_t u_sb;
    const float* dl; int64_t dl_sb;
    const float* A; int64_t A_sd, A_sn;
    const float* Bm; int64_t B_sb, B_sn;
    const float* Cm; int64_t C_sb, C_sn;
    const float* Dv;
    const float* z; int64_t z_sb;
    const float* dbias; bool softplus;
    float* h;  // [nb, D, N] contiguous, in place
    float* y; int64_t y_sb;
};

// Same evaluation as the selective-scan kernel: x above 20 is returned as is.
__device__ __forceinline__ float m1s_softplus(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

__device__ __forceinline__ float m1s_delta(const M1StepParams& p, int b, int d) {
    float dv = p.dl[(int64_t)b * p.dl_sb + d];
    if (p.dbias) dv += p.dbias[d];
    return p.softplus ? m1s_softplus(dv) : dv;
}

// grid (ceil(D / (CPB CPT)), nb), 256 threads; LPC = N/4 lanes per channel,
// CPB channels per round, CPT rounds per thread (all loads of the CPT rounds
// are issued before any arithmetic, for memory-level parallelism).
template <int N, int CPT>
__global__ __launch_bounds__(256) void mamba1_step_kernel(M1StepParams p) {
    constexpr int LPC = N / 4;
    constexpr int CPB = 256 / LPC;
    const int b = blockIdx.y;
    const int t = threadIdx.x;
    const int q = t % LPC;
    const int n0 = 4 * q;
    const int dbase = blockIdx.x * CPB * CPT + t / LPC;
    // a lane group shares d (and so its live flag): shuffles stay inside a group
    int dd[CPT];
    bool live[CPT];
    float4 hv[CPT], av[CPT];
    float dv[CPT], uv[CPT], dbv[CPT], Dvv[CPT], zvv[CPT];
    // optional inputs read through a selected pointer (a real element when
    // absent, its value then dropped), so that no load sits under a branch and
    // every load of the CPT rounds is in flight before the first is used
    const bool has_db = p.dbias != nullptr, has_D = p.Dv != nullptr, has_z = p.z != nullptr;
    const bool a_vec = p.A_sn == 1 && (p.A_sd & 3) == 0 && ((uintptr_t)p.A & 15u) == 0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int d_raw = dbase + k * CPB;
        live[k] = d_raw < p.D;
        dd[k] = live[k] ? d_raw : p.D - 1;
        hv[k] = ld_nt4(reinterpret_cast<const float4*>(p.h + ((int64_t)b * p.D + dd[k]) * N) + q);
        if (a_vec) {
            av[k] = *reinterpret_cast<const float4*>(p.A + (int64_t)dd[k] * p.A_sd + n0);
        } else {
            const float* ar = p.A + (int64_t)dd[k] * p.A_sd;
            av[k] = make_float4(ar[(int64_t)n0 * p.A_sn], ar[(int64_t)(n0 + 1) * p.A_sn],
                                ar[(int64_t)(n0 + 2) * p.A_sn], ar[(int64_t)(n0 + 3) * p.A_sn]);
        }
        dv[k] = p.dl[(int64_t)b * p.dl_sb + dd[k]];
        uv[k] = p.u[(int64_t)b * p.u_sb + dd[k]];
        dbv[k] = *(has_db ? p.dbias + dd[k] : p.dl + (int64_t)b * p.dl_sb + dd[k]);
        Dvv[k] = *(has_D ? p.Dv + dd[k] : p.dl + (int64_t)b * p.dl_sb + dd[k]);
        zvv[k] = *(has_z ? p.z + (int64_t)b * p.z_sb + dd[k] : p.dl + (int64_t)b * p.dl_sb + dd[k]);
    }
    // delta = softplus(delta + bias) (Mamba1::ssm_step, mamba1.rs:646) once every load is issued
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        float v = dv[k] + (has_db ? dbv[k] : 0.f);
        dv[k] = p.softplus ? m1s_softplus(v) : v;
    }
    float bb[4], cc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        bb[e] = p.Bm[(int64_t)b * p.B_sb + (int64_t)(n0 + e) * p.B_sn];
        cc[e] = p.Cm[(int64_t)b * p.C_sb + (int64_t)(n0 + e) * p.C_sn];
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        // h <- h exp(delta A) + (delta B) u ; y partial = sum of this lane's h C
        const float d_ = dv[k], u_ = uv[k];
        float4 hn;
        hn.x = hv[k].x * __expf(d_ * av[k].x) + (d_ * bb[0]) * u_;
        hn.y = hv[k].y * __expf(d_ * av[k].y) + (d_ * bb[1]) * u_;
        hn.z = hv[k].z * __expf(d_ * av[k].z) + (d_ * bb[2]) * u_;
        hn.w = hv[k].w * __expf(d_ * av[k].w) + (d_ * bb[3]) * u_;
        // the channel's sum over its LPC lanes, in the group's last lane
        const float acc = group_sum_last<LPC>(hn.x * cc[0] + hn.y * cc[1] + hn.z * cc[2] + hn.w * cc[3]);
        if (!live[k]) continue;
        st_nt4(reinterpret_cast<float4*>(p.h + ((int64_t)b * p.D + dd[k]) * N) + q, hn);
        if (q == LPC - 1) {
            float out = acc + (has_D ? Dvv[k] : 0.f) * u_;
            if (has_z) {
                const float zv = zvv[k];
                out *= zv * __builtin_amdgcn_rcpf(1.f + __expf(-zv));
            }
            p.y[(int64_t)b * p.y_sb + dd[k]] = out;
        }
    }
}

// Measured on the 64-layer config-2 step (dstate 16), interleaved: four
// channels per thread at batch 64 (1 280 workgroups; 1.15 ms against 1.23 /
// 1.35 ms with 2 / 1) and 32 (0.73 ms; 0.75 with 2); two at batch 16 (0.52 ms
// against 0.55 with 4); one at batch 1 (80 workgroups; 0.30 ms against 0.36
// with 4).
#ifndef MAMBA_M1STEP_MIN_GROUPS
#define MAMBA_M1STEP_MIN_GROUPS 512
#endif
constexpr int64_t kM1StepMinGroups = MAMBA_M1STEP_MIN_GROUPS;

// Any dstate: one thread per channel.
__global__ __launch_bounds__(256) void mamba1_step_generic(M1StepParams p) {
    const int b = blockIdx.y;
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= p.D) return;
    const float dv = m1s_delta(p, b, d);
    const float uv = p.u[(int64_t)b * p.u_sb + d];
    float* hrow = p.h + ((int64_t)b * p.D + d) * p.N;
    float acc = 0.f;
    for (int n = 0; n < p.N; ++n) {
        const float a = p.A[(int64_t)d * p.A_sd + (int64_t)n * p.A_sn];
        const float bv = p.Bm[(int64_t)b * p.B_sb + (int64_t)n * p.B_sn];
        const float cv = p.Cm[(int64_t)b * p.C_sb + (int64_t)n * p.C_sn];
        const float hn = hrow[n] * __expf(dv * a) + (dv * bv) * uv;
        hrow[n] = hn;
        acc += hn * cv;
    }
    float out = acc + (p.Dv ? p.Dv[d] : 0.f) * uv;
    if (p.z) {
        const float zv = p.z[(int64_t)b * p.z_sb + d];
        out *= zv / (1.f + __expf(-zv));
    }
    p.y[(int64_t)b * p.y_sb + d] = out;
}

template <int N, int CPT>
static void m1_step_launch(const M1StepParams& p, hipStream_t s) {
    hipLaunchKernelGGL((mamba1_step_kernel<N, CPT>), dim3(ceil_div(p.D, (256 / (N / 4)) * CPT), p.nb), dim3(256), 0, s,
                       p);
}

// ---------------------------------------------------------------------------
// Depthwise causal conv, one step: window[b,c,:] <- (window[b,c,1:], x[b,c]);
// out[b,c] = act(sum_k window[b,c,k] w[c,k] + bias[c]).
// ---------------------------------------------------------------------------
struct ConvStepParams {
    int nb, C, K;
    bool x_bf16, out_bf16, silu;
    const void* x; int64_t x_sb;
    float* state;
    const float* w; const float* bias;
    void* out; int64_t out_sb;
};

template <bool K4>
__global__ __launch_bounds__(256) void conv1d_step_kernel(ConvStepParams p) {
    const int b = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= p.C) return;
    const int64_t xi = (int64_t)b * p.x_sb + c;
    const float xin = p.x_bf16 ? bf16_to_f32(static_cast<const bf16_t*>(p.x)[xi]) : static_cast<const float*>(p.x)[xi];
    float* win = p.state + ((int64_t)b * p.C + c) * p.K;
    const float* w = p.w + (int64_t)c * p.K;
    // the bias with the other loads (a selected pointer: no load under a branch)
    const float bv = *(p.bias ? p.bias + c : w);
    float acc = 0.f;
    if (K4) {  // one 16-byte window and weight row per channel
        const float4 wv = *reinterpret_cast<const float4*>(win);
        const float4 ww = *reinterpret_cast<const float4*>(w);
        const float4 nw = make_float4(wv.y, wv.z, wv.w, xin);
        *reinterpret_cast<float4*>(win) = nw;
        acc = nw.x * ww.x + nw.y * ww.y + nw.z * ww.z + nw.w * ww.w;
    } else {
        for (int k = 0; k + 1 < p.K; ++k) {
            const float v = win[k + 1];
            win[k] = v;
            acc += v * w[k];
        }
        win[p.K - 1] = xin;
        acc += xin * w[p.K - 1];
    }
    if (p.bias) acc += bv;
    if (p.silu) acc = acc * __builtin_amdgcn_rcpf(__expf(-acc) + 1.f);
    const int64_t oi = (int64_t)b * p.out_sb + c;
    if (p.out_bf16)
        static_cast<bf16_t*>(p.out)[oi] = f32_to_bf16(acc);
    else
        static_cast<float*>(p.out)[oi] = acc;
}

}  // namespace mamba

using namespace mamba;

static int m1_step_dispatch(const mamba1_step_args* a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->dim > 0 && a->dstate > 0 && a->dstate <= 1024,
                    "batch, dim >= 1 and dstate in [1, 1024] required");
    MAMBA_CHECK_ARG(a->u && a->delta && a->A && a->B && a->C && a->state && a->y,
                    "u, delta, A, B, C, state and y are required");
    M1StepParams p;
    p.nb = a->batch; p.D = a->dim; p.N = a->dstate;
    p.u = a->u; p.u_sb = a->u_sb; p.dl = a->delta; p.dl_sb = a->delta_sb;
    p.A = a->A; p.A_sd = a->A_sd; p.A_sn = a->A_sn;
    p.Bm = a->B; p.B_sb = a->B_sb; p.B_sn = a->B_sn;
    p.Cm = a->C; p.C_sb = a->C_sb; p.C_sn = a->C_sn;
    p.Dv = a->D; p.z = a->z; p.z_sb = a->z_sb;
    p.dbias = a->delta_bias; p.softplus = a->delta_softplus != 0;
    p.h = a->state; p.y = a->y; p.y_sb = a->y_sb;
    const bool aligned = ((uintptr_t)p.h & 15u) == 0;
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
    if (aligned && (p.N == 16 || p.N == 32 || p.N == 64)) {
        // channels per thread: 4 (every load of four channels in flight before
        // any arithmetic) while that still gives kM1StepMinGroups workgroups,
        // else fewer, so that small batches spread over more CUs
        const int cpb = 256 / (p.N / 4);
        int cpt = 4;
        while (cpt > 1 && (int64_t)ceil_div(p.D, cpb * cpt) * p.nb < kM1StepMinGroups) cpt /= 2;
        switch (p.N * 8 + cpt) {
            case 16 * 8 + 4: m1_step_launch<16, 4>(p, s); break;
            case 16 * 8 + 2: m1_step_launch<16, 2>(p, s); break;
            case 16 * 8 + 1: m1_step_launch<16, 1>(p, s); break;
            case 32 * 8 + 4: m1_step_launch<32, 4>(p, s); break;
            case 32 * 8 + 2: m1_step_launch<32, 2>(p, s); break;
            case 32 * 8 + 1: m1_step_launch<32, 1>(p, s); break;
            case 64 * 8 + 4: m1_step_launch<64, 4>(p, s); break;
            case 64 * 8 + 2: m1_step_launch<64, 2>(p, s); break;
            default: m1_step_launch<64, 1>(p, s); break;
        }
    } else {
        hipLaunchKernelGGL(mamba1_step_generic, dim3(ceil_div(p.D, 256), p.nb), dim3(256), 0, s, p);
    }
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
    return MAMBA_OK;
}

extern "C" int mamba1_scan_step(const mamba1_step_args* a, mamba_stream_t stream) {
    return m1_step_dispatch(a, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba1_scan_step_timed(const mamba1_step_args* a, mamba_stream_t stream, void* ev_start,
                                      void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba1_scan_step_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return m1_step_dispatch(a, (hipStream_t)stream, (hipEvent_t)ev_start, (hipEvent_t)ev_stop);
}

extern "C" int mamba_conv1d_step(const mamba_conv1d_step_args* a, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->channels > 0, "batch and channels must be >= 1");
    MAMBA_CHECK_ARG(a->kernel >= 1 && a->kernel <= 64, "kernel must be in [1, 64]");
    MAMBA_CHECK_ARG(a->x && a->state && a->w && a->out, "x, state, w and out are required");
    MAMBA_CHECK_ARG(a->x_dtype == MAMBA_F32 || a->x_dtype == MAMBA_BF16, "bad x_dtype");
    MAMBA_CHECK_ARG(a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16, "bad out_dtype");
    ConvStepParams p;
    p.nb = a->batch; p.C = a->channels; p.K = a->kernel;
    p.x_bf16 = a->x_dtype == MAMBA_BF16; p.out_bf16 = a->out_dtype == MAMBA_BF16; p.silu = a->silu != 0;
    p.x = a->x; p.x_sb = a->x_sb; p.state = a->state; p.w = a->w; p.bias = a->bias;
    p.out = a->out; p.out_sb = a->out_sb;
    const bool k4 = p.K == 4 && ((uintptr_t)p.state & 15u) == 0 && ((uintptr_t)p.w & 15u) == 0;
    if (k4)
        hipLaunchKernelGGL(conv1d_step_kernel<true>, dim3(ceil_div(p.C, 256), p.nb), dim3(256), 0, (hipStream_t)stream, p);
    else
        hipLaunchKernelGGL(conv1d_step_kernel<false>, dim3(ceil_div(p.C, 256), p.nb), dim3(256), 0, (hipStream_t)stream, p);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}
