// Mamba-2 recurrent decode step for gfx950: the part of Mamba2::step between
// in_proj and out_proj (burn-mamba src/mamba2/mamba2.rs:857-995), plus the
// residual + RmsNorm of the pre-norm Layer (src/modules/layer.rs:224-232).
//
// The step is HBM-bound: per token and head it streams the f32 state
// [headdim, dstate] in and out once (64 KB at P=64, N=128) and does ~6 flops
// per state element, so there is no MFMA here.  Two kernels per call:
//
//   step2_ssm_*     one workgroup per (batch row, head).  Issues the state
//                   loads first, then slides this head's x-channel conv
//                   windows in place and convolves the group's B/C channels
//                   from their (old) windows, updates the state with
//                   coalesced float4 traffic, reduces y = sum_n h C across the
//                   lanes of each state row with a reduce-scatter (8 partial
//                   rows per lane -> one), gates by z, and writes the gated
//                   values plus a per-(row, head) sum of squares to the
//                   workspace.
//   step2_finish    one workgroup per (1024-channel slice, batch row):
//                   finishes the row's RMS from the per-head partials and
//                   writes out; slice 0 also slides the shared B/C conv
//                   windows.  That slide cannot live in step2_ssm: every head
//                   of a group reads the old B/C window, and kernel order on
//                   the stream is what makes the in-place update safe.
//
// HBM layout: the caches are the reference's Mamba2Cache tensors unchanged
// (conv_bvk [b, conv_dim, K] f32 and ssm_bhpr [b, H, P, N] f32, cache.rs:98-122),
// so a state tile of one (b, h) is one contiguous P*N*4-byte block.
#include <mutex>

#include "common.h"
#include "lin.h"

namespace mamba {

struct Step2Params {
    int nb, H, P, G, N, K, d_inner, conv_dim, hpg;
    bool zx_bf16, out_bf16, norm_before_gate;
    const void* zx; int64_t zx_sb;
    float* conv; const float* conv_w; const float* conv_b;
    const float* dt_bias; const float* A; const float* Dv;
    float dt_lo, dt_hi;
    const float* norm_w;
    float* ssm;
    void* out; int64_t out_sb;
    float* g_ws;    // [nb, d_inner]  gated (or raw, if norm_before_gate) y
    float* ssq_ws;  // [nb, H]        sum of squares of g_ws per head
    // packed mode (the fused layer step): instead of g_ws, write the out_proj
    // operand g * norm_w (norm_before_gate: y * norm_w * silu(z)) in bf16, in
    // the packed activation layout of lin.h with MT = a_mt; the 1/rms of the
    // row is applied after the product (it is a per-row scalar).
    bf16_t* a_out; int a_mt;
    // zxbcdt as zx_S f32 partial planes [zx_S][nb][zx_ld] (+ zx_bias), summed on
    // read; zx_S = 0 reads the single buffer zx (bf16/f32) instead
    const float* zx_part; int zx_S; int64_t zx_ld; const float* zx_bias;
};

// zxbcdt[b, i]: the single buffer, or the sum of the in_proj partial planes.
// ZS > 0: exactly ZS planes, their loads issued together; ZS = 0: p.zx_S at run time.
template <int ZS = 0>
__device__ __forceinline__ float zx_at(const Step2Params& p, const char* zrow, int b, int i) {
    if (ZS == 0 && p.zx_S == 0)
        return p.zx_bf16 ? bf16_to_f32(reinterpret_cast<const bf16_t*>(zrow)[i]) : reinterpret_cast<const float*>(zrow)[i];
    float v = p.zx_bias ? p.zx_bias[i] : 0.f;
    if (ZS > 0) {
        float q[ZS > 0 ? ZS : 1];
#pragma unroll
        for (int s = 0; s < ZS; ++s) q[s] = p.zx_part[((int64_t)s * p.nb + b) * p.zx_ld + i];
#pragma unroll
        for (int s = 0; s < ZS; ++s) v += q[s];
    } else {
        for (int s = 0; s < p.zx_S; ++s) v += p.zx_part[((int64_t)s * p.nb + b) * p.zx_ld + i];
    }
    return v;
}

__device__ __forceinline__ float ld_act(const void* base, int64_t i, bool bf16) {
    return bf16 ? bf16_to_f32(static_cast<const bf16_t*>(base)[i]) : static_cast<const float*>(base)[i];
}

// SiLU with the hardware reciprocal (1 ulp) in place of an IEEE division
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(__expf(-x) + 1.f); }

// dt = clamp(softplus(dt_raw + dt_bias), lo, hi), mamba2.rs:924 with the f32
// softplus threshold of src/modules/activation/softplus.rs:21-47.
template <int ZS = 0>
__device__ __forceinline__ float step_dt(const Step2Params& p, const char* zrow, int b, int h) {
    float v = zx_at<ZS>(p, zrow, b, p.d_inner + p.conv_dim + h);
    if (p.dt_bias) v += p.dt_bias[h];
    float dt = v > 18.f ? v : log1pf(__expf(v));
    return fminf(fmaxf(dt, p.dt_lo), p.dt_hi);
}

// Sum over the 256 threads of a workgroup; every thread gets the result.
__device__ __forceinline__ float block_sum_256(float v, float* s_red) {
    v = wave_sum_dpp(v);  // every thread of the workgroup calls this
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // s_red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) s_red[wave] = v;
    __syncthreads();
    return s_red[0] + s_red[1] + s_red[2] + s_red[3];
}

// ---------------------------------------------------------------------------
// Fast path: headdim 64, dstate N in {64, 128}, conv width 4, 256 threads.
// Thread t owns float4 column n4 = t % (N/4) of rows row0 + i*RPI, i < R.
// RS > 1 (the packed layer path, few batch rows): RS workgroups per (row,
// head), each owning PR = 64 / RS state rows, so that a batch of one still
// launches hundreds of workgroups; each writes its own sum of squares
// (ssq_ws[(b H + h) RS + rs]).
// ---------------------------------------------------------------------------
template <int N, bool PACK, int ZS = 0, int RS = 1>
__global__ __launch_bounds__(256) void step2_ssm_fast(Step2Params p) {
    constexpr int P = 64;
    constexpr int PR = P / RS;      // state rows of this workgroup
    constexpr int LPR = N / 4;      // lanes per state row
    constexpr int RPI = 256 / LPR;  // rows covered by one pass of the workgroup
    constexpr int R = PR / RPI;     // float4 per thread
    static_assert(RS == 1 ? R * 4 == LPR : R >= 1 && PR >= 8, "reduce-scatter assumes R = LPR / 4");
    static_assert(RS == 1 || PACK, "row splits are for the packed layer path");
    __shared__ float s_x[PR];
    __shared__ __align__(16) float s_B[N];
    __shared__ __align__(16) float s_C[N];
    __shared__ float s_red[4];
    __shared__ __align__(16) float s_pk[PACK ? PR : 1];

    const int t = threadIdx.x;
    const int bh = RS == 1 ? (int)blockIdx.x : (int)blockIdx.x / RS;
    const int rs = RS == 1 ? 0 : (int)blockIdx.x % RS, r0 = rs * PR;
    const int b = bh / p.H, h = bh - b * p.H;
    const int g = h / p.hpg;
    const int n4 = t % LPR, row0 = t / LPR;

    // 1. this row's inputs first, into registers: conv windows, weights, the new
    //    inputs (summed in_proj partial planes) and the raw dt.  The conv below
    //    waits for them only, while the state tile (issued next) is in flight.
    const char* zrow = static_cast<const char*>(p.zx) + b * p.zx_sb * (p.zx_bf16 ? 2 : 4);
    float4* win_base = reinterpret_cast<float4*>(p.conv) + (int64_t)b * p.conv_dim;
    const float4* cw = reinterpret_cast<const float4*>(p.conv_w);
    constexpr int CI = (PR + 2 * N + 255) / 256;  // conv channels per thread
    int chs[CI];
    float4 cwin[CI], cwt[CI];
    float cxin[CI], cbias[CI];
#pragma unroll
    for (int j = 0; j < CI; ++j) {
        const int c = min(t + 256 * j, PR + 2 * N - 1);  // clamped: the duplicate is not used
        int ch;
        if (c < PR) ch = h * P + r0 + c;
        else if (c < PR + N) ch = p.d_inner + g * N + (c - PR);
        else ch = p.d_inner + (p.G + g) * N + (c - PR - N);
        chs[j] = ch;
        cwin[j] = win_base[ch];
        cwt[j] = cw[ch];
        cxin[j] = zx_at<ZS>(p, zrow, b, p.d_inner + ch);
        cbias[j] = p.conv_b ? p.conv_b[ch] : 0.f;
    }
    const float dt_raw = zx_at<ZS>(p, zrow, b, p.d_inner + p.conv_dim + h) + (p.dt_bias ? p.dt_bias[h] : 0.f);

    // 2. the state tile: the bytes that matter (read and written once: non-temporal)
    float4* st = reinterpret_cast<float4*>(p.ssm) + (int64_t)bh * (P * LPR) + r0 * LPR;
    float4 hv[R];
#pragma unroll
    for (int i = 0; i < R; ++i) hv[i] = ld_nt4(&st[(row0 + i * RPI) * LPR + n4]);

    // 3. causal conv, one channel per thread (mamba2.rs:865-902)
#pragma unroll
    for (int j = 0; j < CI; ++j) {
        const int c = t + 256 * j;
        if (c >= PR + 2 * N) break;
        const int ch = chs[j];
        const float4 win = cwin[j], w = cwt[j];
        const float xin = cxin[j];
        float acc = win.y * w.x;
        acc += win.z * w.y;
        acc += win.w * w.z;
        acc += xin * w.w;
        acc += cbias[j];
        const float v = silu_fast(acc);
        if (c < PR) {
            s_x[c] = v;
            win_base[ch] = make_float4(win.y, win.z, win.w, xin);
        } else if (c < PR + N) {
            s_B[c - PR] = v;
        } else {
            s_C[c - PR - N] = v;
        }
    }
    // dt = clamp(softplus(dt_raw + dt_bias), lo, hi), mamba2.rs:924 with the f32
    // softplus threshold of src/modules/activation/softplus.rs:21-47
    const float dt = fminf(fmaxf(dt_raw > 18.f ? dt_raw : log1pf(__expf(dt_raw)), p.dt_lo), p.dt_hi);
    const float dA = __expf(dt * p.A[h]);
    const float Dh = p.Dv ? p.Dv[h] : 0.f;
    __syncthreads();

    // 3. h <- h dA + (dt B) x ; partial y per row over this lane's 4 states
    const float4 B4 = reinterpret_cast<const float4*>(s_B)[n4];
    const float4 C4 = reinterpret_cast<const float4*>(s_C)[n4];
    const float4 dB = make_float4(dt * B4.x, dt * B4.y, dt * B4.z, dt * B4.w);
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const float xv = s_x[row0 + i * RPI];
        float4 hn;
        hn.x = hv[i].x * dA + dB.x * xv;
        hn.y = hv[i].y * dA + dB.y * xv;
        hn.z = hv[i].z * dA + dB.z * xv;
        hn.w = hv[i].w * dA + dB.w * xv;
        st_nt4(&st[(row0 + i * RPI) * LPR + n4], hn);
        v[i] = hn.x * C4.x + hn.y * C4.y + hn.z * C4.z + hn.w * C4.w;
    }

    // 5. y = C.h + D x, gate, write gated value and its square (row pr of the
    //    workgroup, ysum its C.h)
    float sq = 0.f;
    auto finish_row = [&](int pr, float ysum) {
        const float y = ysum + Dh * s_x[pr];
        const int ci = h * P + r0 + pr;  // channel
        float gv = y;
        if (PACK) {
            const float zg = silu_fast(zx_at<ZS>(p, zrow, b, ci));
            if (!p.norm_before_gate) gv *= zg;
            s_pk[pr] = p.norm_before_gate ? y * p.norm_w[ci] * zg : gv * p.norm_w[ci];
        } else {
            if (!p.norm_before_gate) gv *= silu_fast(zx_at<ZS>(p, zrow, b, ci));
            p.g_ws[(int64_t)b * p.d_inner + ci] = gv;
        }
        sq += gv * gv;
    };
    if (RS == 1) {
        // 4. reduce-scatter over the LPR lanes of each row group: at xor distance
        //    s the lane with bit s set keeps the upper half of its partials.  After
        //    log2(R) steps lane n4 holds row index (n4 >> 2), summed over 8 lanes;
        //    two more butterflies finish the sum over all LPR lanes.
#pragma unroll
        for (int half = R / 2, s = 2 * R; half >= 1; half >>= 1, s >>= 1) {
            const bool up = (n4 & s) != 0;
#pragma unroll
            for (int j = 0; j < half; ++j) {
                const float keep = up ? v[j + half] : v[j];
                const float send = up ? v[j] : v[j + half];
                v[j] = keep + __shfl_xor(send, s, 64);
            }
        }
        float ysum = v[0];
        ysum += __shfl_xor(ysum, 2, 64);
        ysum += __shfl_xor(ysum, 1, 64);
        if ((n4 & 3) == 0) finish_row(row0 + (n4 >> 2) * RPI, ysum);
    } else {
        // 4'. R rows per thread: each row's sum over its LPR lanes by DPP, in
        //     the row's last lane
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = group_sum_last<LPR>(v[i]);
        if (n4 == LPR - 1)
#pragma unroll
            for (int i = 0; i < R; ++i) finish_row(row0 + i * RPI, v[i]);
    }
    sq = block_sum_256(sq, s_red);  // its barriers also publish s_pk
    if (t == 0) p.ssq_ws[(int64_t)bh * RS + rs] = sq;
    if (PACK && t < PR / 8) {
        // 8 consecutive channels are one 16-byte run of the packed layout
        const float4 lo = reinterpret_cast<const float4*>(s_pk)[2 * t];
        const float4 hi = reinterpret_cast<const float4*>(s_pk)[2 * t + 1];
        uint4 v;
        v.x = (uint32_t)f32_to_bf16(lo.x) | ((uint32_t)f32_to_bf16(lo.y) << 16);
        v.y = (uint32_t)f32_to_bf16(lo.z) | ((uint32_t)f32_to_bf16(lo.w) << 16);
        v.z = (uint32_t)f32_to_bf16(hi.x) | ((uint32_t)f32_to_bf16(hi.y) << 16);
        v.w = (uint32_t)f32_to_bf16(hi.z) | ((uint32_t)f32_to_bf16(hi.w) << 16);
        *reinterpret_cast<uint4*>(p.a_out + lin_act_offset(b, h * P + r0 + 8 * t, p.a_mt)) = v;
    }
}

// ---------------------------------------------------------------------------
// Shape-generic path: any headdim/dstate/conv width; one workgroup per
// (batch row, head), rows over waves, states over lanes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void step2_ssm_generic(Step2Params p) {
    extern __shared__ float s_dyn[];  // [P + 2N]
    __shared__ float s_red[4];
    float* s_x = s_dyn;
    float* s_B = s_dyn + p.P;
    float* s_C = s_B + p.N;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int bh = blockIdx.x;
    const int b = bh / p.H, h = bh - b * p.H;
    const int g = h / p.hpg;
    const int P = p.P, N = p.N, K = p.K;
    const char* zrow = static_cast<const char*>(p.zx) + b * p.zx_sb * (p.zx_bf16 ? 2 : 4);
    for (int c = t; c < P + 2 * N; c += 256) {
        int ch;
        if (c < P) ch = h * P + c;
        else if (c < P + N) ch = p.d_inner + g * N + (c - P);
        else ch = p.d_inner + (p.G + g) * N + (c - P - N);
        float* win = p.conv + ((int64_t)b * p.conv_dim + ch) * K;
        const float* w = p.conv_w + (int64_t)ch * K;
        const float xin = zx_at(p, zrow, b, p.d_inner + ch);
        float acc = 0.f;
        for (int k = 0; k + 1 < K; ++k) acc += win[k + 1] * w[k];
        acc += xin * w[K - 1];
        if (p.conv_b) acc += p.conv_b[ch];
        const float v = silu_fast(acc);
        if (c < P) {
            s_x[c] = v;
            for (int k = 0; k + 1 < K; ++k) win[k] = win[k + 1];
            win[K - 1] = xin;
        } else if (c < P + N) {
            s_B[c - P] = v;
        } else {
            s_C[c - P - N] = v;
        }
    }
    const float dt = step_dt(p, zrow, b, h);
    const float dA = __expf(dt * p.A[h]);
    const float Dh = p.Dv ? p.Dv[h] : 0.f;
    __syncthreads();
    float sq = 0.f;
    for (int pr = wave; pr < P; pr += 4) {
        float* row = p.ssm + ((int64_t)bh * P + pr) * N;
        const float xv = s_x[pr];
        float acc = 0.f;
        for (int n = lane; n < N; n += 64) {
            const float hn = row[n] * dA + (dt * s_B[n]) * xv;
            row[n] = hn;
            acc += hn * s_C[n];
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            const float y = acc + Dh * xv;
            float gv = y;
            if (!p.norm_before_gate) gv *= silu_fast(zx_at(p, zrow, b, h * P + pr));
            p.g_ws[(int64_t)b * p.d_inner + h * P + pr] = gv;
            sq += gv * gv;
        }
    }
    sq = block_sum_256(sq, s_red);
    if (t == 0) p.ssq_ws[bh] = sq;
}

// ---------------------------------------------------------------------------
// Row RMS + normalisation (rms_norm_gated.rs:70-135) and the B/C window slide.
// grid (ceil(d_inner / 1024), nb), 256 threads.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void step2_finish(Step2Params p) {
    __shared__ float s_red[4];
    const int b = blockIdx.y, t = threadIdx.x;
    float s = 0.f;
    for (int i = t; i < p.H; i += 256) s += p.ssq_ws[(int64_t)b * p.H + i];
    s = block_sum_256(s, s_red);
    const float rms = sqrtf(s / (float)p.d_inner + kDivEpsF32);
    const char* zrow = static_cast<const char*>(p.zx) + b * p.zx_sb * (p.zx_bf16 ? 2 : 4);
    const int i0 = blockIdx.x * 1024;
    const int i1 = min(p.d_inner, i0 + 1024);
    for (int i = i0 + t; i < i1; i += 256) {
        float v = (p.g_ws[(int64_t)b * p.d_inner + i] / rms) * p.norm_w[i];
        if (p.norm_before_gate) v *= silu_fast(ld_act(zrow, i, p.zx_bf16));
        if (p.out_bf16)
            static_cast<bf16_t*>(p.out)[b * p.out_sb + i] = f32_to_bf16(v);
        else
            static_cast<float*>(p.out)[b * p.out_sb + i] = v;
    }
    if (blockIdx.x == 0) {
        const int nbc = 2 * p.G * p.N;
        for (int c = t; c < nbc; c += 256) {
            const int ch = p.d_inner + c;
            float* win = p.conv + ((int64_t)b * p.conv_dim + ch) * p.K;
            const float xin = ld_act(zrow, p.d_inner + ch, p.zx_bf16);
            for (int k = 0; k + 1 < p.K; ++k) win[k] = win[k + 1];
            win[p.K - 1] = xin;
        }
    }
}

// ---------------------------------------------------------------------------
// Residual add + RmsNorm: one workgroup per row.
// ---------------------------------------------------------------------------
struct RmsParams {
    int rows, cols;
    bool add_bf16, out_bf16;
    float* x; int64_t x_sr;
    const void* add; int64_t add_sr;
    const float* w;
    void* out; int64_t out_sr;
};

__global__ __launch_bounds__(256) void rmsnorm_residual(RmsParams p) {
    __shared__ float s_red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    float* x = p.x + (int64_t)r * p.x_sr;
    float ss = 0.f;
    for (int c = t; c < p.cols; c += 256) {
        float v = x[c];
        if (p.add) {
            v += ld_act(p.add, (int64_t)r * p.add_sr + c, p.add_bf16);
            x[c] = v;
        }
        ss += v * v;
    }
    if (!p.out) return;
    ss = block_sum_256(ss, s_red);
    const float rms = sqrtf(ss / (float)p.cols + kDivEpsF32);
    for (int c = t; c < p.cols; c += 256) {
        const float v = (x[c] / rms) * p.w[c];
        if (p.out_bf16)
            static_cast<bf16_t*>(p.out)[(int64_t)r * p.out_sr + c] = f32_to_bf16(v);
        else
            static_cast<float*>(p.out)[(int64_t)r * p.out_sr + c] = v;
    }
}

// The same with the row in registers, a float4 per thread and step (V steps:
// cols <= 1024 V), every load of the row issued before any arithmetic (one
// memory round trip instead of a load per column step and a second pass over
// x).  Needs cols % 4 == 0 and 16-byte rows (8-byte for bf16 operands); the
// per-element arithmetic is the scalar kernel's.
template <int V>
__global__ __launch_bounds__(256) void rmsnorm_residual_v(RmsParams p) {
    __shared__ float s_red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    const int nv = p.cols >> 2;
    float4* x = reinterpret_cast<float4*>(p.x + (int64_t)r * p.x_sr);
    float4 v[V], a[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c4 = t + 256 * i;
        const bool in = c4 < nv;
        v[i] = in ? x[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        a[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p.add && in) {
            if (p.add_bf16) {
                const uint2 u = reinterpret_cast<const uint2*>(static_cast<const bf16_t*>(p.add) + (int64_t)r * p.add_sr)[c4];
                a[i] = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                                   __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
            } else {
                a[i] = reinterpret_cast<const float4*>(static_cast<const float*>(p.add) + (int64_t)r * p.add_sr)[c4];
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c4 = t + 256 * i;
        if (p.add) {
            v[i].x += a[i].x; v[i].y += a[i].y; v[i].z += a[i].z; v[i].w += a[i].w;
            if (c4 < nv) x[c4] = v[i];
        }
        ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    if (!p.out) return;
    ss = block_sum_256(ss, s_red);
    const float rms = sqrtf(ss / (float)p.cols + kDivEpsF32);
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c4 = t + 256 * i;
        if (c4 >= nv) continue;
        const float4 w4 = reinterpret_cast<const float4*>(p.w)[c4];
        const float4 o = make_float4((v[i].x / rms) * w4.x, (v[i].y / rms) * w4.y, (v[i].z / rms) * w4.z,
                                     (v[i].w / rms) * w4.w);
        if (p.out_bf16) {
            reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.out) + (int64_t)r * p.out_sr)[c4] =
                make_uint2((uint32_t)f32_to_bf16(o.x) | ((uint32_t)f32_to_bf16(o.y) << 16),
                           (uint32_t)f32_to_bf16(o.z) | ((uint32_t)f32_to_bf16(o.w) << 16));
        } else {
            reinterpret_cast<float4*>(static_cast<float*>(p.out) + (int64_t)r * p.out_sr)[c4] = o;
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static size_t step2_ws_bytes(const mamba2_step_args* a) {
    const size_t d_inner = (size_t)a->nheads * a->headdim;
    return align_up((size_t)a->batch * d_inner * 4, 256) + align_up((size_t)a->batch * a->nheads * 4, 256);
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

static int step2_make_params(const mamba2_step_args* a, void* ws, size_t ws_bytes, Step2Params* out) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->nheads > 0 && a->headdim > 0 && a->ngroups > 0 && a->dstate > 0,
                    "batch, nheads, headdim, ngroups and dstate must be >= 1");
    MAMBA_CHECK_ARG(a->nheads % a->ngroups == 0, "nheads must be divisible by ngroups");
    MAMBA_CHECK_ARG(a->conv_kernel >= 1 && a->conv_kernel <= 16, "conv_kernel must be in [1, 16]");
    MAMBA_CHECK_ARG(a->zxbcdt_dtype == MAMBA_F32 || a->zxbcdt_dtype == MAMBA_BF16, "bad zxbcdt_dtype");
    MAMBA_CHECK_ARG(a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16, "bad out_dtype");
    MAMBA_CHECK_ARG(a->zxbcdt && a->conv_state && a->conv_w && a->A && a->norm_w && a->ssm_state && a->out,
                    "zxbcdt, conv_state, conv_w, A, norm_w, ssm_state and out are required");
    const int64_t d_inner = (int64_t)a->nheads * a->headdim;
    const int64_t conv_dim = d_inner + 2ll * a->ngroups * a->dstate;
    MAMBA_CHECK_ARG(d_inner + conv_dim + a->nheads < (1ll << 30), "row too long");
    MAMBA_CHECK_ARG(a->zxbcdt_sb >= d_inner + conv_dim + a->nheads, "zxbcdt_sb shorter than a row");
    MAMBA_CHECK_ARG(a->out_sb >= d_inner, "out_sb shorter than a row");
    MAMBA_CHECK_ARG(!(a->dt_min > a->dt_max), "dt_min > dt_max");
    const size_t need = step2_ws_bytes(a);
    if (ws == nullptr || ws_bytes < need) {
        set_error("mamba2_step_ssm: workspace of " + std::to_string(need) + " bytes required, got " +
                  std::to_string(ws == nullptr ? 0 : ws_bytes));
        return MAMBA_ERR_WORKSPACE;
    }
    Step2Params& p = *out;
    p.nb = a->batch; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups; p.N = a->dstate;
    p.K = a->conv_kernel; p.d_inner = (int)d_inner; p.conv_dim = (int)conv_dim; p.hpg = p.H / p.G;
    p.zx_bf16 = a->zxbcdt_dtype == MAMBA_BF16; p.out_bf16 = a->out_dtype == MAMBA_BF16;
    p.norm_before_gate = a->norm_before_gate != 0;
    p.zx = a->zxbcdt; p.zx_sb = a->zxbcdt_sb;
    p.conv = a->conv_state; p.conv_w = a->conv_w; p.conv_b = a->conv_b;
    p.dt_bias = a->dt_bias; p.A = a->A; p.Dv = a->D;
    p.dt_lo = a->dt_min; p.dt_hi = a->dt_max;
    p.norm_w = a->norm_w; p.ssm = a->ssm_state;
    p.out = a->out; p.out_sb = a->out_sb;
    p.g_ws = static_cast<float*>(ws);
    p.ssq_ws = reinterpret_cast<float*>(static_cast<char*>(ws) + align_up((size_t)p.nb * d_inner * 4, 256));
    p.a_out = nullptr; p.a_mt = 0;
    p.zx_part = nullptr; p.zx_S = 0; p.zx_ld = 0; p.zx_bias = nullptr;
    return MAMBA_OK;
}

static int step2_dispatch(const mamba2_step_args* a, void* ws, size_t ws_bytes, hipStream_t stream,
                          hipEvent_t ev0, hipEvent_t ev1) {
    Step2Params p;
    int st = step2_make_params(a, ws, ws_bytes, &p);
    if (st != MAMBA_OK) return st;
    const bool fast = p.P == 64 && (p.N == 64 || p.N == 128) && p.K == 4 && aligned16(p.ssm) &&
                      aligned16(p.conv) && aligned16(p.conv_w);
    const dim3 grid(p.nb * p.H);
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    if (fast && p.N == 128)
        hipLaunchKernelGGL((step2_ssm_fast<128, false>), grid, dim3(256), 0, stream, p);
    else if (fast)
        hipLaunchKernelGGL((step2_ssm_fast<64, false>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(step2_ssm_generic, grid, dim3(256), (p.P + 2 * p.N) * sizeof(float), stream, p);
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    hipLaunchKernelGGL(step2_finish, dim3(ceil_div(p.d_inner, 1024), p.nb), dim3(256), 0, stream, p);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

extern "C" size_t mamba2_step_workspace_size(const mamba2_step_args* a) {
    return a ? step2_ws_bytes(a) : 0;
}

extern "C" int mamba2_step_ssm(const mamba2_step_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream) {
    return step2_dispatch(a, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba2_step_ssm_timed(const mamba2_step_args* a, void* ws, size_t ws_bytes,
                                     mamba_stream_t stream, void* ev_start, void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba2_step_ssm_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return step2_dispatch(a, ws, ws_bytes, (hipStream_t)stream, (hipEvent_t)ev_start, (hipEvent_t)ev_stop);
}

extern "C" int mamba_rmsnorm(const mamba_rmsnorm_args* a, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->rows > 0 && a->cols > 0, "rows and cols must be >= 1");
    MAMBA_CHECK_ARG(a->x != nullptr, "x is required");
    MAMBA_CHECK_ARG(a->add || a->out, "nothing to do: add and out are both NULL");
    MAMBA_CHECK_ARG(!a->out || a->weight, "weight is required with out");
    MAMBA_CHECK_ARG(a->add_dtype == MAMBA_F32 || a->add_dtype == MAMBA_BF16, "bad add_dtype");
    MAMBA_CHECK_ARG(a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16, "bad out_dtype");
    MAMBA_CHECK_ARG(a->x_sr >= a->cols && (!a->add || a->add_sr >= a->cols) && (!a->out || a->out_sr >= a->cols),
                    "row strides shorter than cols");
    RmsParams p;
    p.rows = a->rows; p.cols = a->cols;
    p.add_bf16 = a->add_dtype == MAMBA_BF16; p.out_bf16 = a->out_dtype == MAMBA_BF16;
    p.x = a->x; p.x_sr = a->x_sr; p.add = a->add; p.add_sr = a->add_sr;
    p.w = a->weight; p.out = a->out; p.out_sr = a->out_sr;
    // the register form where every row is 16-byte aligned (8-byte for bf16)
    auto rows_ok = [](const void* ptr, int64_t sr, bool bf16) {
        return ptr == nullptr || (((uintptr_t)ptr & (bf16 ? 7u : 15u)) == 0 && sr % 4 == 0);
    };
    const bool vec = p.cols % 4 == 0 && p.cols <= 4096 && rows_ok(p.x, p.x_sr, false) &&
                     rows_ok(p.add, p.add_sr, p.add_bf16) && rows_ok(p.out, p.out_sr, p.out_bf16) &&
                     (p.out == nullptr || ((uintptr_t)p.w & 15u) == 0);
    const hipStream_t s = (hipStream_t)stream;
    if (!vec) hipLaunchKernelGGL(rmsnorm_residual, dim3(p.rows), dim3(256), 0, s, p);
    else if (p.cols <= 1024) hipLaunchKernelGGL(rmsnorm_residual_v<1>, dim3(p.rows), dim3(256), 0, s, p);
    else if (p.cols <= 2048) hipLaunchKernelGGL(rmsnorm_residual_v<2>, dim3(p.rows), dim3(256), 0, s, p);
    else if (p.cols <= 3072) hipLaunchKernelGGL(rmsnorm_residual_v<3>, dim3(p.rows), dim3(256), 0, s, p);
    else hipLaunchKernelGGL(rmsnorm_residual_v<4>, dim3(p.rows), dim3(256), 0, s, p);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

// ---------------------------------------------------------------------------
// Fused pre-norm layer step: x += out_proj(RmsNormGated(ssm(in_proj(RmsNorm(x)))))
// and the whole stack of them.
// ---------------------------------------------------------------------------
namespace mamba {

// One workgroup per row m of the residual stream x[m, 0:cols):
//   S > 0:  x += (sum of the S out_proj planes) / rms_ssq(m) (+ bias), where
//           rms_ssq(m) = sqrt(sum_h ssq[m, h] / d_inner + eps) finishes the
//           gated RMSNorm of the layer just computed, and the shared B/C conv
//           windows of row m slide (every head has read them by now);
//   PACK:   write RmsNorm(x)[m, :] * w (rms_norm.rs:53-98) in bf16, packed as
//           the next in_proj operand.
// Every thread keeps its columns in registers between the two parts.
struct RowsParams {
    int M, cols, H, d_inner, conv_dim, conv_k, nbc;  // nbc: B/C channels (2 G N)
    int nssq;  // sum-of-squares partials per row (heads x state-kernel row splits)
    float* x; int64_t x_ld;
    const float* part; const float* bias; const float* ssq;
    float* conv; const float* zx_part; int zx_S; int64_t zx_ld; const float* zx_bias;
    const float* w; bf16_t* a_out; int a_mt;
};

constexpr int kRowsThreads = 1024;  // a row per workgroup: one float4 per thread, more loads in flight
constexpr int kRowsMaxVec = 1;      // float4 per thread: cols <= 4096
constexpr int kRowsMaxHeads = 256;
__device__ __forceinline__ float block_sum_rows(float v, float* s_red) {
    v = wave_sum_dpp(v);  // every thread of the workgroup calls this
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kRowsThreads / 64; ++w) s += s_red[w];
    return s;
}

// Workgroups past the M row workgroups slide the shared B/C conv windows of
// the layer just computed (every head has read them by now): one thread per
// (row, B/C channel), all of its loads issued together.
__device__ __forceinline__ void bc_window_slide(const RowsParams& p, int idx) {
    if (idx >= p.M * p.nbc) return;
    const int m = idx / p.nbc, c = idx - m * p.nbc;
    const int ch = p.d_inner + c;
    float4* win = reinterpret_cast<float4*>(p.conv + ((int64_t)m * p.conv_dim + ch) * 4);
    const float4 old = *win;
    const int zi = p.d_inner + ch;
    float zs[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) zs[z] = z < p.zx_S ? p.zx_part[((int64_t)z * p.M + m) * p.zx_ld + zi] : 0.f;
    float xin = p.zx_bias ? p.zx_bias[zi] : 0.f;
#pragma unroll
    for (int z = 0; z < 16; ++z) xin += zs[z];
    *win = make_float4(old.y, old.z, old.w, xin);
}

template <int S, bool PACK>
__global__ __launch_bounds__(kRowsThreads) void layer_rows(RowsParams p) {
    __shared__ float s_red[kRowsThreads / 64];
    if (S > 0 && (int)blockIdx.x >= p.M) {
        bc_window_slide(p, ((int)blockIdx.x - p.M) * kRowsThreads + (int)threadIdx.x);
        return;
    }
    const int m = blockIdx.x, t = threadIdx.x;
    const int nv = p.cols / 4;
    float4* xr = reinterpret_cast<float4*>(p.x + (int64_t)m * p.x_ld);
    // ---- every load of this row first (one memory round trip) ----
    float4 v[kRowsMaxVec], acc[kRowsMaxVec], bb[kRowsMaxVec], w4[kRowsMaxVec];
#pragma unroll
    for (int i = 0; i < kRowsMaxVec; ++i) {
        const int c4 = t + i * kRowsThreads;
        const bool in = c4 < nv;
        v[i] = in ? xr[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        bb[i] = (S > 0 && in && p.bias) ? reinterpret_cast<const float4*>(p.bias)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        w4[i] = (PACK && in) ? reinterpret_cast<const float4*>(p.w)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float4 q[S > 0 ? S : 1][kRowsMaxVec];
#pragma unroll
    for (int z = 0; z < S; ++z) {
        const float4* pl = reinterpret_cast<const float4*>(p.part + ((int64_t)z * p.M + m) * p.cols);
#pragma unroll
        for (int i = 0; i < kRowsMaxVec; ++i) {
            const int c4 = t + i * kRowsThreads;
            q[z][i] = c4 < nv ? pl[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float ss_h = 0.f;
    if (S > 0 && t < p.nssq) ss_h = p.ssq[(int64_t)m * p.nssq + t];
    if (S > 0) {
        // ---- residual of the layer just computed ----
        const float rms = sqrtf(block_sum_rows(ss_h, s_red) / (float)p.d_inner + kDivEpsF32);
#pragma unroll
        for (int z = 0; z < S; ++z)
#pragma unroll
            for (int i = 0; i < kRowsMaxVec; ++i) {
                acc[i].x += q[z][i].x; acc[i].y += q[z][i].y; acc[i].z += q[z][i].z; acc[i].w += q[z][i].w;
            }
#pragma unroll
        for (int i = 0; i < kRowsMaxVec; ++i) {
            const int c4 = t + i * kRowsThreads;
            v[i].x += acc[i].x / rms + bb[i].x;
            v[i].y += acc[i].y / rms + bb[i].y;
            v[i].z += acc[i].z / rms + bb[i].z;
            v[i].w += acc[i].w / rms + bb[i].w;
            if (c4 < nv) xr[c4] = v[i];
        }
    }
    if (PACK) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kRowsMaxVec; ++i) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
        const float rms = sqrtf(block_sum_rows(ss, s_red) / (float)p.cols + kDivEpsF32);
        // lanes 2q and 2q+1 hold columns 8q..8q+7 of a slab: one 16-byte run of
        // the packed operand, written by the even lane
#pragma unroll
        for (int i = 0; i < kRowsMaxVec; ++i) {
            const int c4 = t + i * kRowsThreads;
            const uint32_t lo = (uint32_t)f32_to_bf16((v[i].x / rms) * w4[i].x) |
                                ((uint32_t)f32_to_bf16((v[i].y / rms) * w4[i].y) << 16);
            const uint32_t hi = (uint32_t)f32_to_bf16((v[i].z / rms) * w4[i].z) |
                                ((uint32_t)f32_to_bf16((v[i].w / rms) * w4[i].w) << 16);
            const uint32_t lo_n = __shfl_xor(lo, 1, 64), hi_n = __shfl_xor(hi, 1, 64);
            if (c4 < nv && (c4 & 1) == 0)
                *reinterpret_cast<uint4*>(p.a_out + lin_act_offset(m, 4 * c4, p.a_mt)) = make_uint4(lo, hi, lo_n, hi_n);
        }
    }
}

template <bool PACK>
static void rows_launch(const RowsParams& rp, int S, hipStream_t stream) {
    const dim3 g(rp.M + (S > 0 ? (rp.M * rp.nbc + kRowsThreads - 1) / kRowsThreads : 0)), b(kRowsThreads);
    switch (S) {
        case 0: hipLaunchKernelGGL((layer_rows<0, PACK>), g, b, 0, stream, rp); break;
        case 1: hipLaunchKernelGGL((layer_rows<1, PACK>), g, b, 0, stream, rp); break;
        case 2: hipLaunchKernelGGL((layer_rows<2, PACK>), g, b, 0, stream, rp); break;
        case 4: hipLaunchKernelGGL((layer_rows<4, PACK>), g, b, 0, stream, rp); break;
        case 8: hipLaunchKernelGGL((layer_rows<8, PACK>), g, b, 0, stream, rp); break;
        default: hipLaunchKernelGGL((layer_rows<16, PACK>), g, b, 0, stream, rp); break;
    }
}

struct LayerGeom {
    int M, d_model, H, d_inner, conv_dim, d_in_proj, nbc, mt, S_in, S_out, nw_in, nw_out;
    int rs;  // state-kernel workgroups per (row, head)
};

// Row splits of the state kernel: with few batch rows, one workgroup per
// (row, head) leaves most CUs idle (80 workgroups at batch 1 for the 2.7B
// layer), so each head's 64 state rows are shared by up to 8 workgroups, until
// the launch has at least kStep2MinGroups of them.
constexpr int kStep2MinGroups = 512;
static int step2_row_splits(int rows, int heads, int N) {
    const int cap = N == 128 ? 8 : 4;  // R >= 1 float4 per thread, 8 rows per workgroup
    int rs = 1;
    while (rs < cap && rows * heads * rs < kStep2MinGroups) rs *= 2;
    return rs;
}

// Products of a call that runs beside another stream's layers (a batch split
// over two streams) with one 32-row tile: in_proj with one k-split and 8 waves
// per workgroup, out_proj with two k-splits and 16 waves.  Measured on the
// 64-layer config-3 step at batch 64 (two 32-row halves): 6.04 -> 5.88 ms; the
// same plan on one stream at batch 32 measured 2.8 % slower than lin_splits'.
#ifndef MAMBA_STEP2_CC_S_IN
#define MAMBA_STEP2_CC_S_IN 1
#endif
#ifndef MAMBA_STEP2_CC_NW_IN
#define MAMBA_STEP2_CC_NW_IN 8
#endif
#ifndef MAMBA_STEP2_CC_S_OUT
#define MAMBA_STEP2_CC_S_OUT 2
#endif
#ifndef MAMBA_STEP2_CC_NW_OUT
#define MAMBA_STEP2_CC_NW_OUT 16
#endif

// Products of a one-stream call with one row tile: in_proj two k-splits of 8
// waves (up to 32 rows), and at one row (lin_gemv) out_proj two of 16, in
// place of lin_splits' 4 and 8 of 4 waves.  Measured on the 64-layer config-3
// step: batch 1 1.89 -> 1.86 ms (each change alone about 1 %; one k-split, or 8
// in_proj k-splits, slower); the in_proj plan at batch 8 / 16 / 24 2.50 /
// 3.01 / 3.52 -> 2.47 / 2.97 / 3.48 ms, where the out_proj one did not pay.
#ifndef MAMBA_STEP2_R1_ROWS
#define MAMBA_STEP2_R1_ROWS 32
#endif
#ifndef MAMBA_STEP2_R1_OUT_ROWS
#define MAMBA_STEP2_R1_OUT_ROWS 1
#endif
#ifndef MAMBA_STEP2_R1_S_IN
#define MAMBA_STEP2_R1_S_IN 2
#endif
#ifndef MAMBA_STEP2_R1_NW_IN
#define MAMBA_STEP2_R1_NW_IN 8
#endif
#ifndef MAMBA_STEP2_R1_S_OUT
#define MAMBA_STEP2_R1_S_OUT 2
#endif
#ifndef MAMBA_STEP2_R1_NW_OUT
#define MAMBA_STEP2_R1_NW_OUT 16
#endif

struct LayerWs {
    bf16_t* a_in; float* zx_part; bf16_t* a_out; float* ssq; float* out_part; size_t total;
};

static LayerGeom layer_geom(const mamba2_layer_args* a) {
    LayerGeom g;
    g.M = a->batch; g.d_model = a->d_model; g.H = a->nheads;
    g.d_inner = a->nheads * a->headdim;
    g.nbc = 2 * a->ngroups * a->dstate;
    g.conv_dim = g.d_inner + g.nbc;
    g.d_in_proj = g.d_inner + g.conv_dim + g.H;
    g.mt = lin_mt(g.M);
    g.S_in = lin_splits(g.M, g.d_model, g.d_in_proj);
    g.S_out = lin_splits(g.M, g.d_inner, g.d_model);
    g.rs = step2_row_splits(g.M, g.H, a->dstate);
    g.nw_in = g.nw_out = 0;
    if (a->concurrent && g.mt == 1) {
        g.S_in = MAMBA_STEP2_CC_S_IN;
        g.S_out = MAMBA_STEP2_CC_S_OUT;
        g.nw_in = MAMBA_STEP2_CC_NW_IN;
        g.nw_out = MAMBA_STEP2_CC_NW_OUT;
    } else if (g.mt == 1 && g.M <= MAMBA_STEP2_R1_ROWS) {
        if (MAMBA_STEP2_R1_S_IN) g.S_in = MAMBA_STEP2_R1_S_IN;
        if (MAMBA_STEP2_R1_NW_IN) g.nw_in = MAMBA_STEP2_R1_NW_IN;
        if (g.M <= MAMBA_STEP2_R1_OUT_ROWS) {
            if (MAMBA_STEP2_R1_S_OUT) g.S_out = MAMBA_STEP2_R1_S_OUT;
            if (MAMBA_STEP2_R1_NW_OUT) g.nw_out = MAMBA_STEP2_R1_NW_OUT;
        }
    }
    return g;
}

static LayerWs layer_ws_layout(const LayerGeom& g, void* base) {
    char* p = static_cast<char*>(base);
    LayerWs w;
    size_t off = 0;
    auto take = [&](size_t bytes) { char* q = p + off; off += align_up(bytes, 256); return q; };
    w.a_in = reinterpret_cast<bf16_t*>(take(lin_act_elems(g.M, g.d_model) * 2));
    w.zx_part = reinterpret_cast<float*>(take(lin_part_elems(g.M, g.d_in_proj, g.S_in) * 4));
    w.a_out = reinterpret_cast<bf16_t*>(take(lin_act_elems(g.M, g.d_inner) * 2));
    w.ssq = reinterpret_cast<float*>(take((size_t)g.M * g.H * g.rs * 4));
    w.out_part = reinterpret_cast<float*>(take(lin_part_elems(g.M, g.d_model, g.S_out) * 4));
    w.total = off;
    return w;
}

// Validates one layer's arguments against the geometry of the first.
static int layer_check(const mamba2_layer_args* a, const mamba2_layer_args* first) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch >= 1 && a->batch <= 256, "batch must be in [1, 256]");
    MAMBA_CHECK_ARG(a->d_model > 0 && a->d_model % 16 == 0 && a->d_model <= 4 * kRowsMaxVec * kRowsThreads,
                    "d_model must be a positive multiple of 16, at most 4096");
    // layer_rows reduces the per-head sums of squares with one thread per head
    MAMBA_CHECK_ARG(a->nheads >= 1 && a->nheads <= kRowsMaxHeads, "nheads must be in [1, 256]");
    MAMBA_CHECK_ARG(a->x && a->pre_norm_w && a->in_proj && a->out_proj, "x, pre_norm_w, in_proj, out_proj required");
    MAMBA_CHECK_ARG(a->x_sb >= a->d_model && a->x_sb % 4 == 0, "x_sb must be >= d_model and a multiple of 4");
    if (!(a->headdim == 64 && (a->dstate == 64 || a->dstate == 128) && a->conv_kernel == 4)) {
        set_error("mamba2_layer_step: needs headdim 64, dstate 64 or 128 and conv_kernel 4 "
                  "(use mamba2_step_ssm with a separate product otherwise)");
        return MAMBA_ERR_UNSUPPORTED;
    }
    MAMBA_CHECK_ARG(aligned16(a->in_proj) && aligned16(a->out_proj) && aligned16(a->x) && aligned16(a->pre_norm_w) &&
                    (!a->out_proj_b || aligned16(a->out_proj_b)),
                    "packed weights, x, pre_norm_w and out_proj_b must be 16-byte aligned");
    MAMBA_CHECK_ARG(aligned16(a->ssm_state) && aligned16(a->conv_state) && aligned16(a->conv_w),
                    "ssm_state, conv_state and conv_w must be 16-byte aligned");
    if (first && a != first) {
        MAMBA_CHECK_ARG(a->batch == first->batch && a->d_model == first->d_model && a->nheads == first->nheads &&
                            a->headdim == first->headdim && a->ngroups == first->ngroups &&
                            a->dstate == first->dstate && a->conv_kernel == first->conv_kernel &&
                            a->x == first->x && a->x_sb == first->x_sb && a->concurrent == first->concurrent,
                        "every layer of a stack must share the shapes and the residual stream x");
    }
    return MAMBA_OK;
}

// in_proj, state update, out_proj of one layer; a_in must hold the packed
// normed input.  Leaves the out_proj planes and ssq in the workspace.
static int layer_core(const mamba2_layer_args* a, const LayerGeom& g, const LayerWs& w, hipStream_t stream,
                      hipEvent_t ev0, hipEvent_t ev1) {
    LinParams li = {};
    li.M = g.M; li.N = g.d_in_proj; li.K = g.d_model; li.MT = g.mt; li.S = g.S_in; li.NW = g.nw_in;
    li.W = static_cast<const lin_bf16x8_t*>(a->in_proj);
    li.A = reinterpret_cast<const lin_bf16x8_t*>(w.a_in);
    li.part = w.zx_part;
    lin_launch(li, LIN_PARTIAL, stream);
    MAMBA_CHECK_LAUNCH();

    mamba2_step_args sa = {};
    sa.batch = a->batch; sa.nheads = a->nheads; sa.headdim = a->headdim; sa.ngroups = a->ngroups;
    sa.dstate = a->dstate; sa.conv_kernel = a->conv_kernel;
    sa.zxbcdt_dtype = MAMBA_F32; sa.out_dtype = MAMBA_BF16; sa.norm_before_gate = a->norm_before_gate;
    sa.zxbcdt = w.zx_part; sa.zxbcdt_sb = g.d_in_proj;
    sa.conv_state = a->conv_state; sa.conv_w = a->conv_w; sa.conv_b = a->conv_b;
    sa.dt_bias = a->dt_bias; sa.A = a->A; sa.D = a->D; sa.dt_min = a->dt_min; sa.dt_max = a->dt_max;
    sa.norm_w = a->norm_w; sa.ssm_state = a->ssm_state;
    sa.out = w.a_out; sa.out_sb = g.d_inner;  // validated only: the packed path writes a_out itself
    Step2Params p;
    int st = step2_make_params(&sa, w.ssq, (size_t)-1 >> 1, &p);  // no step workspace in packed mode
    if (st != MAMBA_OK) return st;
    p.g_ws = nullptr; p.ssq_ws = w.ssq;
    p.a_out = w.a_out; p.a_mt = g.mt;
    p.zx_part = w.zx_part; p.zx_S = g.S_in; p.zx_ld = g.d_in_proj; p.zx_bias = a->in_proj_b;
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    const dim3 kg(p.nb * p.H * g.rs), kb(256);
#define MAMBA_STEP2_PACKED(NN, RS)                                                                     \
    switch (g.S_in) {                                                                                  \
        case 1: hipLaunchKernelGGL((step2_ssm_fast<NN, true, 1, RS>), kg, kb, 0, stream, p); break;    \
        case 2: hipLaunchKernelGGL((step2_ssm_fast<NN, true, 2, RS>), kg, kb, 0, stream, p); break;    \
        case 4: hipLaunchKernelGGL((step2_ssm_fast<NN, true, 4, RS>), kg, kb, 0, stream, p); break;    \
        default: hipLaunchKernelGGL((step2_ssm_fast<NN, true, 0, RS>), kg, kb, 0, stream, p); break;   \
    }
    if (p.N == 128) {
        switch (g.rs) {
            case 1: MAMBA_STEP2_PACKED(128, 1) break;
            case 2: MAMBA_STEP2_PACKED(128, 2) break;
            case 4: MAMBA_STEP2_PACKED(128, 4) break;
            default: MAMBA_STEP2_PACKED(128, 8) break;
        }
    } else {
        switch (g.rs) {
            case 1: MAMBA_STEP2_PACKED(64, 1) break;
            case 2: MAMBA_STEP2_PACKED(64, 2) break;
            default: MAMBA_STEP2_PACKED(64, 4) break;
        }
    }
#undef MAMBA_STEP2_PACKED
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));

    LinParams lo = {};
    lo.M = g.M; lo.N = g.d_model; lo.K = g.d_inner; lo.MT = g.mt; lo.S = g.S_out; lo.NW = g.nw_out;
    lo.W = static_cast<const lin_bf16x8_t*>(a->out_proj);
    lo.A = reinterpret_cast<const lin_bf16x8_t*>(w.a_out);
    lo.part = w.out_part;
    lin_launch(lo, LIN_PARTIAL, stream);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

static RowsParams rows_params(const mamba2_layer_args* a, const LayerGeom& g, const LayerWs& w) {
    RowsParams rp = {};
    rp.M = g.M; rp.cols = g.d_model; rp.H = g.H; rp.d_inner = g.d_inner; rp.conv_dim = g.conv_dim;
    rp.nssq = g.H * g.rs;
    rp.conv_k = a->conv_kernel; rp.nbc = g.nbc;
    rp.x = a->x; rp.x_ld = a->x_sb;
    rp.part = w.out_part; rp.bias = a->out_proj_b; rp.ssq = w.ssq;
    rp.conv = a->conv_state; rp.zx_part = w.zx_part; rp.zx_S = g.S_in; rp.zx_ld = g.d_in_proj;
    rp.zx_bias = a->in_proj_b;
    rp.a_out = w.a_in; rp.a_mt = g.mt;
    return rp;
}

// n_layers consecutive layers on one residual stream; events (optional) are
// per-layer arrays recorded around each state-update kernel.
static int stack_dispatch(const mamba2_layer_args* layers, int n_layers, void* ws, size_t ws_bytes,
                          hipStream_t stream, void* const* ev0, void* const* ev1) {
    MAMBA_CHECK_ARG(layers != nullptr && n_layers >= 1, "at least one layer is required");
    for (int l = 0; l < n_layers; ++l) {
        const int st = layer_check(&layers[l], &layers[0]);
        if (st != MAMBA_OK) return st;
    }
    const LayerGeom g = layer_geom(&layers[0]);
    const LayerWs w = layer_ws_layout(g, ws);
    if (ws == nullptr || ws_bytes < w.total) {
        set_error("mamba2 layer step: workspace of " + std::to_string(w.total) + " bytes required");
        return MAMBA_ERR_WORKSPACE;
    }
    // pre-norm of the first layer
    RowsParams rp = rows_params(&layers[0], g, w);
    rp.w = layers[0].pre_norm_w;
    rows_launch<true>(rp, 0, stream);
    MAMBA_CHECK_LAUNCH();
    for (int l = 0; l < n_layers; ++l) {
        const mamba2_layer_args* a = &layers[l];
        const int st = layer_core(a, g, w, stream, ev0 ? (hipEvent_t)ev0[l] : nullptr,
                                  ev1 ? (hipEvent_t)ev1[l] : nullptr);
        if (st != MAMBA_OK) return st;
        // residual of layer l, fused with the pre-norm of layer l + 1
        rp = rows_params(a, g, w);
        if (l + 1 < n_layers) {
            rp.w = layers[l + 1].pre_norm_w;
            rows_launch<true>(rp, g.S_out, stream);
        } else {
            rows_launch<false>(rp, g.S_out, stream);
        }
        MAMBA_CHECK_LAUNCH();
    }
    return MAMBA_OK;
}

// ------------------------------------------------ allocation-free stack --
// The workspace of mamba2_stack_step_noalloc: a file-scope device array.  Each
// GPU the library runs on holds its own copy (at its own address) until the
// process ends.  Host code never passes `scratch` itself to a kernel or a copy:
// on the host the name is only a stand-in for the symbol, so the device address
// of the current GPU's copy is looked up once per device and kept.
static __device__ __align__(256) unsigned char scratch[MAMBA2_STACK_NOALLOC_SCRATCH_BYTES];

constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchDevices] = {};

// Device address of the current GPU's `scratch` (looked up on the first call
// on that device, with that device current).
static int scratch_address(void** out) {
    int dev = -1;
    MAMBA_CHECK_HIP(hipGetDevice(&dev));
    MAMBA_CHECK_ARG(dev >= 0 && dev < kScratchDevices, "device index out of range for the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        MAMBA_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        MAMBA_CHECK_ARG(ptr != nullptr && ((uintptr_t)ptr & 255u) == 0, "scratch symbol address is not usable");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MAMBA_OK;
}

}  // namespace mamba

extern "C" int mamba2_stack_step_noalloc(const mamba2_layer_args* layers, int32_t n_layers, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(layers != nullptr && n_layers >= 1, "at least one layer is required");
    const int st = layer_check(&layers[0], &layers[0]);
    if (st != MAMBA_OK) return st;
    const size_t need = layer_ws_layout(layer_geom(&layers[0]), nullptr).total;
    if (need > MAMBA2_STACK_NOALLOC_SCRATCH_BYTES) {
        set_error("mamba2_stack_step_noalloc: this stack needs a workspace of " + std::to_string(need) +
                  " bytes, more than the " + std::to_string(MAMBA2_STACK_NOALLOC_SCRATCH_BYTES) +
                  "-byte scratch array; use mamba2_stack_step with a caller workspace");
        return MAMBA_ERR_WORKSPACE;
    }
    void* ws = nullptr;
    const int sa = scratch_address(&ws);
    if (sa != MAMBA_OK) return sa;
    // every workspace region is written before it is read within the call
    // (packed operands, partial planes, per-head sums), so nothing is cleared
    return stack_dispatch(layers, n_layers, ws, MAMBA2_STACK_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream, nullptr,
                          nullptr);
}

extern "C" size_t mamba2_layer_workspace_size(const mamba2_layer_args* a) {
    if (a == nullptr || a->batch < 1 || a->nheads < 1 || a->headdim < 1) return 0;
    return layer_ws_layout(layer_geom(a), nullptr).total;
}

extern "C" int mamba2_layer_step(const mamba2_layer_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream) {
    return stack_dispatch(a, 1, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba2_layer_step_timed(const mamba2_layer_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream,
                                       void* ev_start, void* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba2_layer_step_timed: both events are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return stack_dispatch(a, 1, ws, ws_bytes, (hipStream_t)stream, &ev_start, &ev_stop);
}

extern "C" int mamba2_stack_step(const mamba2_layer_args* layers, int32_t n_layers, void* ws, size_t ws_bytes,
                                 mamba_stream_t stream) {
    return stack_dispatch(layers, n_layers, ws, ws_bytes, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int mamba2_stack_step_timed(const mamba2_layer_args* layers, int32_t n_layers, void* ws, size_t ws_bytes,
                                       mamba_stream_t stream, void* const* ev_start, void* const* ev_stop) {
    if (ev_start == nullptr || ev_stop == nullptr) {
        set_error("mamba2_stack_step_timed: both event arrays are required");
        return MAMBA_ERR_INVALID_ARG;
    }
    return stack_dispatch(layers, n_layers, ws, ws_bytes, (hipStream_t)stream, ev_start, ev_stop);
}
