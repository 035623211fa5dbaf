// Mamba-3 recurrent decode step for gfx950: everything of Mamba3::step between
// in_proj and out_proj, one workgroup per (batch row, head).
//
// Reference: Mamba3::step_double_ssd (burn-mamba
// src/mamba3/double_ssd/double_ssd/mod.rs:634-760): step_project (:407-496:
// split, trapezoidal_coefficients helpers.rs:42-73, qk_norm_expand_bias
// helpers.rs:82-95), rotate_bc_step Complex2D (rotation/mod.rs:729-763 with
// angle_increment :559-567, wrap_angle / apply_rope_partial rope.rs:23-170),
// build_v_with_mimo + mimo_outer_sum (helpers.rs:113-168), step_readout
// (mod.rs:516-550) and step_finish without out_proj (mod.rs:556-628).
// Single-SSD decoding uses the same step (single_ssd/single_ssd/mod.rs:383-397).
//
// Per (b, h), with v[m,p] = x[p] mimo_x[h,m,p] and xs[m,p] = v_state[p] mimo_x[h,m,p]:
//   h      <- alpha h + sum_m gamma v[m] (x) B[m] + sum_m beta xs[m] (x) K[m]
//   out[m] = sum_n C[m,n] h[p,n] + D v[m,p]
//   y[p]   = sum_m mimo_o[h,m,p] G(out[m,p], z[p] mimo_z[h,m,p])   (M = 1: G(out, z))
// with B, C QK-normed, biased and rotated by the cumulative angle, K the
// previous token's rotated B, G the silu gate or the per-head gated RMSNorm.
// The state tile (P x N f32) is read and written once: the step is HBM-bound.
#include "mamba3_internal.h"

namespace mamba {

struct M3StepParams {
    int nb, H, P, G, N, M, R, A;  // R = rope_dim, A = angles per head
    bool proj_bf16, out_bf16;
    const void* proj; int64_t proj_sb;
    float* ssm; float* kst; float* vst; float* ang;
    const float* dt_bias; float a_floor, dt_lo, dt_hi, span;
    const float* bnw; const float* cnw; const float* bbias; const float* cbias;
    const float* mx; const float* mz; const float* mo;
    const float* Dh; const float* onw;
    void* out; int64_t out_sb;
};

constexpr int kM3MaxPN = 8192;  // state tile elements held in registers (P*N)

__device__ __forceinline__ float m3_silu(float x) { return x * m3_sigmoid(x); }

__device__ __forceinline__ float m3_proj(const M3StepParams& p, const void* row, int i) {
    return p.proj_bf16 ? bf16_to_f32(static_cast<const bf16_t*>(row)[i]) : static_cast<const float*>(row)[i];
}

// wrap_angle: subtract round-half-even(a / 2pi) 2pi (rope.rs:23-27)
__device__ __forceinline__ float m3_wrap(float a) {
    const float two_pi = 6.28318530717958647692f;
    return a - rintf(a * (1.f / two_pi)) * two_pi;
}

// N4 = N/4 lanes per state row (a power of two, <= 64); MM = MIMO rank.
template <int N4, int MM>
__global__ __launch_bounds__(256) void mamba3_step_kernel(M3StepParams p) {
    constexpr int N = 4 * N4;
    constexpr int RPP = 256 / N4;                  // state rows per pass
    constexpr int MAXPASS = kM3MaxPN / (RPP * N);  // register budget of the prefetch
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int q = t % N4, row0 = t / N4;
    const int P = p.P;
    const int npass = (P + RPP - 1) / RPP;
    const int64_t bh = (int64_t)b * p.H + h;
    float* st = p.ssm + bh * P * N;

    // the readout's row sums: QS lanes by DPP, then SL partials per row and
    // rank through LDS (row pitch padded by one word)
    constexpr int QS = N4 < 4 ? N4 : 4, SL = N4 / QS, PS = SL * MM + 1;
    constexpr int PMAX = kM3MaxPN / N < 256 ? kM3MaxPN / N : 256;
    __shared__ __align__(16) float s_B[MM][N], s_C[MM][N], s_K[MM][N];
    __shared__ float s_gv[MM][256], s_bx[MM][256], s_v[MM][256], s_out[MM][256];
    __shared__ float s_part[PMAX * PS];
    __shared__ float s_cs[128], s_sn[128], s_rms[2 * MM], s_coef[3];

    const void* row = static_cast<const char*>(p.proj) + (int64_t)b * p.proj_sb * (p.proj_bf16 ? 2 : 4);
    const int d_inner = p.H * P, bc = MM * p.G * N;
    const int o_b = 2 * d_inner, o_c = o_b + bc, o_dt = o_c + bc, o_a = o_dt + p.H, o_l = o_a + p.H,
              o_rot = o_l + p.H;
    const int g = h / (p.H / p.G);
    // B/C rows in rotation pairs, (k, k + N/2) for MIMO > 1 and (2k, 2k + 1)
    // for MIMO 1 (rotate_bc_step): a row's N/2 pairs over a group of GS lanes
    // (PPL pairs per lane), RPI rows per pass of the workgroup, JR passes
    constexpr int NP = N / 2, GS = NP < 64 ? NP : 64, PPL = NP / GS;
    constexpr int NROW = 2 * MM, RPI = 256 / GS, JR = (NROW + RPI - 1) / RPI;
    const int gl = t % GS, rsub = t / GS;
    // ---- this row's inputs first, into registers: the prep below waits for
    // them only, while the state tile (issued next) is still in flight
    constexpr int RK = (MM * N + 255) / 256;
    const float raw_dt = m3_proj(p, row, o_dt + h), raw_a = m3_proj(p, row, o_a + h),
                raw_l = m3_proj(p, row, o_l + h), dtb = p.dt_bias[h];
    float raw_rot = 0.f, ang0 = 0.f;
    if (t < p.A) {
        raw_rot = m3_proj(p, row, o_rot + t);
        ang0 = p.ang[bh * p.A + t];
    }
    // raw B/C pair values, their norm weights and this head's biases
    float x0[JR][PPL], x1[JR][PPL], w0[JR][PPL], w1[JR][PPL], c0[JR][PPL], c1[JR][PPL];
#pragma unroll
    for (int j = 0; j < JR; ++j) {
        const int r = rsub + RPI * j;
        const bool in = r < NROW;
        const int rr = in ? r : 0, wh = rr / MM, mm = rr % MM;
        const int src = (wh ? o_c : o_b) + (mm * p.G + g) * N;
        const float* nw = wh ? p.cnw : p.bnw;
        const float* bias = (wh ? p.cbias : p.bbias) + ((int64_t)h * MM + mm) * N;
#pragma unroll
        for (int e = 0; e < PPL; ++e) {
            const int k = gl * PPL + e, i0 = MM == 1 ? 2 * k : k, i1 = MM == 1 ? 2 * k + 1 : k + NP;
            x0[j][e] = in ? m3_proj(p, row, src + i0) : 0.f;
            x1[j][e] = in ? m3_proj(p, row, src + i1) : 0.f;
            w0[j][e] = nw[i0]; w1[j][e] = nw[i1];
            c0[j][e] = bias[i0]; c1[j][e] = bias[i1];
        }
    }
    float rk[RK];
#pragma unroll
    for (int j = 0; j < RK; ++j) {
        const int i = t + 256 * j, m = i / N, n = i % N;
        rk[j] = i < MM * N ? p.kst[(((int64_t)b * MM + m) * p.H + h) * N + n] : 0.f;
    }
    float xv = 0.f, xo = 0.f, mxv[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) mxv[m] = 1.f;
    if (t < P) {
        xv = m3_proj(p, row, d_inner + h * P + t);
        xo = p.vst[bh * P + t];
        if (p.mx)
#pragma unroll
            for (int m = 0; m < MM; ++m) mxv[m] = p.mx[((int64_t)h * MM + m) * P + t];
    }

    // ---- the state tile: unconditional loads (rows clamped into the tile, the
    // duplicates unused), so the waits on the inputs above are exact counts
    float4 hv[MAXPASS];
#pragma unroll
    for (int k = 0; k < MAXPASS; ++k) {
        const int pr = min(row0 + k * RPP, P - 1);
        hv[k] = ld_nt4(reinterpret_cast<const float4*>(st + (int64_t)pr * N) + q);
    }
    // the gate's inputs, issued after the tile (first used after the update)
    float zq = 0.f, onq = 0.f, mzq[MM], moq[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        mzq[m] = 1.f;
        moq[m] = 1.f;
    }
    if (t < P) {
        zq = m3_proj(p, row, h * P + t);
        if (p.onw) onq = p.onw[t];
        if (MM > 1)
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                mzq[m] = p.mz[((int64_t)h * MM + m) * P + t];
                moq[m] = p.mo[((int64_t)h * MM + m) * P + t];
            }
    }

    // ---- trapezoid coefficients and the cumulative angle, on the waves that
    // hold angles (wave 0 at least); the others read the coefficients from LDS
    // (the prefill's arithmetic: hardware exp / reciprocal / sin / cos)
    if (wave * 64 < (p.A > 64 ? p.A : 64)) {
        float dt, da, lam;
        m3_coef(raw_dt, raw_a, raw_l, dtb, p.a_floor, p.dt_lo, p.dt_hi, dt, da, lam);
        if (t == 0) {
            const float alpha = __expf(da);
            s_coef[0] = alpha;
            s_coef[1] = (1.f - lam) * dt * alpha;  // beta
            s_coef[2] = lam * dt;                  // gamma
        }
        if (t < p.A) {
            const float th = m3_wrap(ang0 + m3_angle_inc(dt, raw_rot, p.span));
            p.ang[bh * p.A + t] = th;
            if (t < 128) m3_cossin(m3_wrap(th), s_cs[t], s_sn[t]);
        }
    }
    // ---- the previous token's K; QK-norm of the B/C rows (sum of squares over
    // the row's lane group), weight and bias, in registers
#pragma unroll
    for (int j = 0; j < RK; ++j) {
        const int i = t + 256 * j, m = i / N, n = i % N;
        if (i < MM * N) s_K[m][n] = rk[j];
    }
#pragma unroll
    for (int j = 0; j < JR; ++j) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < PPL; ++e) ss += x0[j][e] * x0[j][e] + x1[j][e] * x1[j][e];
        ss = group_sum_last<GS>(ss);
        ss = __shfl(ss, (lane & ~(GS - 1)) + GS - 1, 64);
        const float rms = m3_rms_inv(ss, N);
#pragma unroll
        for (int e = 0; e < PPL; ++e) {
            x0[j][e] = m3_norm(x0[j][e], rms, w0[j][e], c0[j][e]);
            x1[j][e] = m3_norm(x1[j][e], rms, w1[j][e], c1[j][e]);
        }
    }
    __syncthreads();
    // ---- rotation of the first R/2 pairs by the angle's cos/sin, into LDS
    const int npair = p.R / 2;
#pragma unroll
    for (int j = 0; j < JR; ++j) {
        const int r = rsub + RPI * j;
        if (r < NROW) {
            const int which = r / MM, m = r % MM;
            float* vv = which ? s_C[m] : s_B[m];
#pragma unroll
            for (int e = 0; e < PPL; ++e) {
                const int k = gl * PPL + e, i0 = MM == 1 ? 2 * k : k, i1 = MM == 1 ? 2 * k + 1 : k + NP;
                float r0 = x0[j][e], r1 = x1[j][e];
                if (k < npair) {
                    const float cs = s_cs[k], sn = s_sn[k];
                    r0 = cs * x0[j][e] - sn * x1[j][e];
                    r1 = sn * x0[j][e] + cs * x1[j][e];
                }
                vv[i0] = r0;
                vv[i1] = r1;
            }
        }
    }
    const float alpha = s_coef[0], beta = s_coef[1], gamma = s_coef[2];
    if (t < P) {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            s_v[m][t] = xv * mxv[m];
            s_gv[m][t] = gamma * (xv * mxv[m]);
            s_bx[m][t] = beta * (xo * mxv[m]);
        }
    }
    __syncthreads();
    // ---- new cache entries: K <- rotated B, v_state <- x (old ones are in LDS)
    for (int i = t; i < MM * N; i += 256) {
        const int m = i / N, n = i % N;
        p.kst[(((int64_t)b * MM + m) * p.H + h) * N + n] = s_B[m][n];
    }
    if (t < P) p.vst[bh * P + t] = xv;

    // ---- state update and readout, N4 lanes per row
    const int n0 = 4 * q;
    float4 bq[MM], kq[MM], cq[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        bq[m] = *reinterpret_cast<const float4*>(&s_B[m][n0]);
        kq[m] = *reinterpret_cast<const float4*>(&s_K[m][n0]);
        cq[m] = *reinterpret_cast<const float4*>(&s_C[m][n0]);
    }
    const float Dv = p.Dh ? p.Dh[h] : 0.f;
#pragma unroll
    for (int k = 0; k < MAXPASS; ++k) {
        const int pr = row0 + k * RPP;
        if (k >= npass) break;
        const bool live = pr < P;
        const int pc = live ? pr : 0;
        float4 hn;
        hn.x = alpha * hv[k].x; hn.y = alpha * hv[k].y; hn.z = alpha * hv[k].z; hn.w = alpha * hv[k].w;
        float acc[MM];
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float gv = s_gv[m][pc], bx = s_bx[m][pc];
            hn.x = __builtin_fmaf(bx, kq[m].x, __builtin_fmaf(gv, bq[m].x, hn.x));
            hn.y = __builtin_fmaf(bx, kq[m].y, __builtin_fmaf(gv, bq[m].y, hn.y));
            hn.z = __builtin_fmaf(bx, kq[m].z, __builtin_fmaf(gv, bq[m].z, hn.z));
            hn.w = __builtin_fmaf(bx, kq[m].w, __builtin_fmaf(gv, bq[m].w, hn.w));
        }
#pragma unroll
        for (int m = 0; m < MM; ++m)
            acc[m] = __builtin_fmaf(cq[m].w, hn.w, __builtin_fmaf(cq[m].z, hn.z, __builtin_fmaf(cq[m].y, hn.y, cq[m].x * hn.x)));
        // the sum over QS lanes lands in the last of them
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[m] = group_sum_last<QS>(acc[m]);
        if (live) {
            st_nt4(reinterpret_cast<float4*>(st + (int64_t)pr * N) + q, hn);
            if (q % QS == QS - 1)
#pragma unroll
                for (int m = 0; m < MM; ++m) s_part[pr * PS + (q / QS) * MM + m] = acc[m];
        }
    }
    __syncthreads();
    // the rows' readout: SL partials per (row, rank), in order
    for (int i = t; i < P * MM; i += 256) {
        const int pr = i / MM, m = i % MM;
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < SL; ++j) sum += s_part[pr * PS + j * MM + m];
        s_out[m][pr] = __builtin_fmaf(Dv, s_v[m][pr], sum);
    }
    __syncthreads();
    // ---- gate (or per-head gated norm over P), MIMO merge
    if (p.onw) {
        for (int m = wave; m < MM; m += 4) {
            float ss = 0.f;
            for (int i = lane; i < P; i += 64) ss += s_out[m][i] * s_out[m][i];
            ss = wave_sum(ss);
            if (lane == 0) s_rms[m] = m3_rms_inv(ss, P);
        }
        __syncthreads();
    }
    if (t < P) {
        const int i = t;
        float y = 0.f;
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float zm = MM > 1 ? zq * mzq[m] : zq;
            float gv = p.onw ? (s_out[m][i] * s_rms[m]) * onq * m3_silu(zm) : s_out[m][i] * m3_silu(zm);
            if (MM > 1) gv *= moq[m];
            y += gv;
        }
        const int64_t oi = (int64_t)b * p.out_sb + h * P + i;
        if (p.out_bf16)
            static_cast<bf16_t*>(p.out)[oi] = f32_to_bf16(y);
        else
            static_cast<float*>(p.out)[oi] = y;
    }
}

template <int N4>
static void m3_launch_m(const M3StepParams& p, hipStream_t s) {
    const dim3 grid(p.nb * p.H), block(256);
    switch (p.M) {
        case 1: hipLaunchKernelGGL((mamba3_step_kernel<N4, 1>), grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL((mamba3_step_kernel<N4, 2>), grid, block, 0, s, p); break;
        case 4: hipLaunchKernelGGL((mamba3_step_kernel<N4, 4>), grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL((mamba3_step_kernel<N4, 8>), grid, block, 0, s, p); break;
    }
}

static int m3_step_dispatch(const mamba3_step_args* a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->nheads > 0 && a->headdim > 0 && a->ngroups > 0, "sizes must be >= 1");
    MAMBA_CHECK_ARG(a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    const int N = a->dstate;
    MAMBA_CHECK_ARG(N == 8 || N == 16 || N == 32 || N == 64 || N == 128 || N == 256,
                    "dstate must be one of 8, 16, 32, 64, 128, 256");
    MAMBA_CHECK_ARG(a->headdim <= 256 && (int64_t)a->headdim * N <= kM3MaxPN,
                    "headdim <= 256 and headdim * dstate <= 8192 required");
    MAMBA_CHECK_ARG(a->mimo == 1 || a->mimo == 2 || a->mimo == 4 || a->mimo == 8, "mimo must be 1, 2, 4 or 8");
    MAMBA_CHECK_ARG(a->rope_dim >= 0 && a->rope_dim <= N && a->rope_dim % 2 == 0 && a->rope_dim / 2 <= 128,
                    "rope_dim must be even and in [0, dstate]");
    MAMBA_CHECK_ARG(a->mimo == 1 || (a->mimo_x && a->mimo_z && a->mimo_o),
                    "mimo_x, mimo_z and mimo_o are required when mimo > 1");
    MAMBA_CHECK_ARG(a->proj && a->ssm_state && a->k_state && a->v_state && a->angle && a->dt_bias &&
                        a->b_norm_w && a->c_norm_w && a->b_bias && a->c_bias && a->out,
                    "proj, the four cache tensors, dt_bias, norm weights, biases and out are required");
    MAMBA_CHECK_ARG(a->proj_dtype == MAMBA_F32 || a->proj_dtype == MAMBA_BF16, "bad proj_dtype");
    MAMBA_CHECK_ARG(a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16, "bad out_dtype");
    MAMBA_CHECK_ARG(((uintptr_t)a->ssm_state & 15u) == 0, "ssm_state must be 16-byte aligned");
    const int A = a->rope_dim / 2 > 1 ? a->rope_dim / 2 : 1;
    const int64_t row = 2LL * a->nheads * a->headdim + 2LL * a->mimo * a->ngroups * N + 3LL * a->nheads + A;
    MAMBA_CHECK_ARG(a->proj_sb >= row, "proj_sb is smaller than the in_proj row");
    MAMBA_CHECK_ARG(a->out_sb >= (int64_t)a->nheads * a->headdim, "out_sb is smaller than d_inner");
    M3StepParams p;
    p.nb = a->batch; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups; p.N = N; p.M = a->mimo;
    p.R = a->rope_dim; p.A = A;
    p.proj_bf16 = a->proj_dtype == MAMBA_BF16; p.out_bf16 = a->out_dtype == MAMBA_BF16;
    p.proj = a->proj; p.proj_sb = a->proj_sb;
    p.ssm = a->ssm_state; p.kst = a->k_state; p.vst = a->v_state; p.ang = a->angle;
    p.dt_bias = a->dt_bias; p.a_floor = a->a_floor; p.dt_lo = a->dt_min; p.dt_hi = a->dt_max;
    p.span = (float)((double)a->rotation_range * 3.14159265358979323846);
    p.bnw = a->b_norm_w; p.cnw = a->c_norm_w; p.bbias = a->b_bias; p.cbias = a->c_bias;
    p.mx = a->mimo_x; p.mz = a->mimo_z; p.mo = a->mimo_o; p.Dh = a->D; p.onw = a->out_norm_w;
    p.out = a->out; p.out_sb = a->out_sb;
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, s));
    switch (N) {
        case 8: m3_launch_m<2>(p, s); break;
        case 16: m3_launch_m<4>(p, s); break;
        case 32: m3_launch_m<8>(p, s); break;
        case 64: m3_launch_m<16>(p, s); break;
        case 128: m3_launch_m<32>(p, s); break;
        default: m3_launch_m<64>(p, s); break;
    }
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, s));
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" int mamba3_step_ssm(const mamba3_step_args* a, mamba_stream_t stream) {
    return m3_step_dispatch(a, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba3_step_ssm_timed(const mamba3_step_args* a, mamba_stream_t stream, void* ev_start,
                                     void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba3_step_ssm_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return m3_step_dispatch(a, (hipStream_t)stream, (hipEvent_t)ev_start, (hipEvent_t)ev_stop);
}
