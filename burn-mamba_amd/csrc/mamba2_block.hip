// Mamba-2 full-block prefill around the SSD seam, gfx950: the prologue after
// in_proj and the epilogue before out_proj.
//
// Reference: Mamba2::forward (burn-mamba src/mamba2/mamba2.rs:546-786).
//  * mamba2_conv_fwd (steps 2 and 4, :618-699): the causal depthwise conv1d
//    over the xBC channels of the in_proj rows, left-padded with the cached
//    window, + bias, SiLU (silu.rs:24-27); dt = softplus(dt_raw + dt_bias)
//    clamped to dt_limit (:695, softplus.rs:17-48).  The conv window of the
//    cache becomes the last `kernel` columns of the padded input
//    (mamba2.rs:652-655); it is updated in place by a second kernel that runs
//    after the first has read the old window.  With nheads = 0 there is no dt
//    and this is the Mamba-1 prefill conv (Mamba1::forward layer 2,
//    src/mamba1/mamba1.rs:300-340: the same padded causal conv, SiLU and
//    window update over the x half of the in_proj rows).
//  * mamba2_gated_rmsnorm (step 7, :776; RmsNormGated, rms_norm_gated.rs:70-135):
//    gate-then-norm (default) or norm-then-gate over a row of `width`,
//    rms = sqrt(mean(x^2) + eps) with the caller's eps (div_eps of the
//    reference's dtype, utils/mod.rs:50-95).
#include "common.h"

namespace mamba {

template <typename T> __device__ __forceinline__ float m2_ld1(const T* q);
template <> __device__ __forceinline__ float m2_ld1<float>(const float* q) { return *q; }
template <> __device__ __forceinline__ float m2_ld1<bf16_t>(const bf16_t* q) { return bf16_to_f32(*q); }
template <typename T> __device__ __forceinline__ void m2_st1(T* q, float v);
template <> __device__ __forceinline__ void m2_st1<float>(float* q, float v) { *q = v; }
template <> __device__ __forceinline__ void m2_st1<bf16_t>(bf16_t* q, float v) { *q = f32_to_bf16(v); }

// SiLU x / (1 + e^-x) (silu.rs:24-27) with the hardware reciprocal (1 ulp)
// in place of an IEEE division; x -> -inf gives x * rcp(inf) = -0.
__device__ __forceinline__ float m2_silu(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// 8 consecutive elements at a 16-byte aligned address
template <typename T> __device__ __forceinline__ void m2_ld8(const T* q, float* o);
template <> __device__ __forceinline__ void m2_ld8<float>(const float* q, float* o) {
    const float4 a = *(const float4*)q, c = *(const float4*)(q + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = c.x; o[5] = c.y; o[6] = c.z; o[7] = c.w;
}
template <> __device__ __forceinline__ void m2_ld8<bf16_t>(const bf16_t* q, float* o) {
    const uint4 u = *(const uint4*)q;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o[2 * k] = __uint_as_float(w[k] << 16);
        o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}
template <typename T> __device__ __forceinline__ void m2_st8(T* q, const float* v);
template <> __device__ __forceinline__ void m2_st8<float>(float* q, const float* v) {
    *(float4*)q = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(q + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
template <> __device__ __forceinline__ void m2_st8<bf16_t>(bf16_t* q, const float* v) {
    *(uint4*)q = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                            pack_bf16x2(v[6], v[7]));
}

struct M2ConvParams {
    int nb, L, V, K, H;
    const void* proj; int64_t proj_sb, proj_sl;
    int xbc_off, dt_off;
    const float* w; const float* bias;
    float* state;
    const float* dt_bias; float dt_lo, dt_hi;
    void* out; int64_t out_sb, out_sl;
    float* dt;
};

constexpr int kM2ConvTile = 64;  // positions per workgroup
constexpr int kM2ConvRows = 8;   // input rows in flight per thread
constexpr int kM2MaxK = 8;

// One thread per VW consecutive channels over a tile of kM2ConvTile positions:
// the last K - 1 inputs stay in registers, so every input is read once.
// Channels c of position l: sum_k w[c][k] xpad[l + k] with xpad = [the
// window's last K - 1 columns | the new inputs].  The channel blocks of a
// tile also share out the tile's dt.
template <typename TI, typename TO, int VW, int K>
__global__ __launch_bounds__(256) void mamba2_conv_kernel(M2ConvParams p) {
    const int tile = blockIdx.x, b = blockIdx.z;
    const int c0 = (blockIdx.y * 256 + threadIdx.x) * VW;
    const int l0 = tile * kM2ConvTile, l1 = min(p.L, l0 + kM2ConvTile);
    const TI* proj = static_cast<const TI*>(p.proj) + (int64_t)b * p.proj_sb;
    if (c0 < p.V) {
        float w[VW][K], bias[VW];
#pragma unroll
        for (int e = 0; e < VW; ++e) {
#pragma unroll
            for (int k = 0; k < K; ++k) w[e][k] = p.w[(int64_t)(c0 + e) * K + k];
            bias[e] = p.bias ? p.bias[c0 + e] : 0.f;
        }
        // window: win[j] holds xpad[l0 + j] for j < K - 1 (positions l0 - K + 1 + j)
        float win[K > 1 ? K - 1 : 1][VW];
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
            const int l = l0 - (K - 1) + j;  // uniform over the workgroup
            bool done = false;
            if constexpr (VW == 8) {
                if (l >= 0) {
                    m2_ld8(proj + (int64_t)l * p.proj_sl + p.xbc_off + c0, win[j]);
                    done = true;
                }
            }
            if (!done) {
#pragma unroll
                for (int e = 0; e < VW; ++e) {
                    float v;
                    if (l >= 0)
                        v = m2_ld1(proj + (int64_t)l * p.proj_sl + p.xbc_off + c0 + e);
                    else  // cache column (K + l): the window's last K - 1 columns end at column K - 1
                        v = p.state[((int64_t)b * p.V + c0 + e) * K + K + l];
                    win[j][e] = v;
                }
            }
        }
        TO* out = static_cast<TO*>(p.out) + (int64_t)b * p.out_sb;
        // one position: convolve, slide the window, store
        auto emit = [&](int l, const float* x) {
            float y[VW];
#pragma unroll
            for (int e = 0; e < VW; ++e) {
                float acc = bias[e];
#pragma unroll
                for (int k = 0; k < K - 1; ++k) acc += w[e][k] * win[k][e];
                acc += w[e][K - 1] * x[e];
                y[e] = m2_silu(acc);
            }
#pragma unroll
            for (int j = 0; j + 1 < K - 1; ++j)
#pragma unroll
                for (int e = 0; e < VW; ++e) win[j][e] = win[j + 1][e];
            if constexpr (K > 1) {
#pragma unroll
                for (int e = 0; e < VW; ++e) win[K - 2][e] = x[e];
            }
            TO* dst = out + (int64_t)l * p.out_sl + c0;
            if constexpr (VW == 8) {
                m2_st8(dst, y);
            } else {
#pragma unroll
                for (int e = 0; e < VW; ++e) m2_st1(dst + e, y[e]);
            }
        };
        auto load = [&](int l, float* x) {
            const TI* src = proj + (int64_t)l * p.proj_sl + p.xbc_off + c0;
            if constexpr (VW == 8) {
                m2_ld8(src, x);
            } else {
#pragma unroll
                for (int e = 0; e < VW; ++e) x[e] = m2_ld1(src + e);
            }
        };
        // kM2ConvRows rows are loaded before any is used, so their HBM
        // latencies overlap instead of adding up row by row
        int l = l0;
        for (; l + kM2ConvRows <= l1; l += kM2ConvRows) {
            float xs[kM2ConvRows][VW];
#pragma unroll
            for (int u = 0; u < kM2ConvRows; ++u) load(l + u, xs[u]);
#pragma unroll
            for (int u = 0; u < kM2ConvRows; ++u) emit(l + u, xs[u]);
        }
        for (; l < l1; ++l) {
            float x[VW];
            load(l, x);
            emit(l, x);
        }
    }
    // the tile's dt, its (position, head) pairs split over the channel blocks;
    // each thread issues all its loads before its stores
    {
        const int n = (l1 - l0) * p.H, per = (n + gridDim.y - 1) / gridDim.y;
        const int i0 = blockIdx.y * per, i1 = min(n, i0 + per);
        constexpr int kU = 4;
        for (int ib = i0 + (int)threadIdx.x; ib < i1; ib += 256 * kU) {
            float raw[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int i = ib + 256 * u;
                raw[u] = i < i1 ? m2_ld1(proj + (int64_t)(l0 + i / p.H) * p.proj_sl + p.dt_off + i % p.H) : 0.f;
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int i = ib + 256 * u;
                if (i < i1) {
                    const int l = l0 + i / p.H, h = i % p.H;
                    const float v = raw[u] + p.dt_bias[h];
                    const float sp = v > 18.f ? v : log1pf(__expf(v));
                    p.dt[((int64_t)b * p.L + l) * p.H + h] = fminf(fmaxf(sp, p.dt_lo), p.dt_hi);
                }
            }
        }
    }
}

// The new window: the last K columns of [old window's last K - 1 | inputs],
// one thread per (batch, channel), in place (all K old values are read first).
template <typename TI>
__global__ __launch_bounds__(256) void mamba2_conv_state_kernel(M2ConvParams p) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)p.nb * p.V) return;
    const int b = (int)(i / p.V), c = (int)(i % p.V);
    const TI* proj = static_cast<const TI*>(p.proj) + (int64_t)b * p.proj_sb;
    float* st = p.state + i * p.K;
    float old[kM2MaxK], nw[kM2MaxK];
    for (int k = 0; k < p.K; ++k) old[k] = st[k];
    // padded column j of the new window: padded index (L - 1) + j; padded
    // index q < K - 1 is old column q + 1, else input position q - (K - 1)
    for (int j = 0; j < p.K; ++j) {
        const int q = p.L - 1 + j;
        nw[j] = q < p.K - 1 ? old[q + 1] : m2_ld1(proj + (int64_t)(q - (p.K - 1)) * p.proj_sl + p.xbc_off + c);
    }
    for (int k = 0; k < p.K; ++k) st[k] = nw[k];
}

struct M2NormParams {
    int nb, L, W;
    bool before;
    float eps;
    const void* y; int64_t y_sb, y_sl;
    const void* z; int64_t z_sb, z_sl;
    const float* gamma;
    void* out; int64_t out_sb, out_sl;
};

// One wave per (b, l) row; lanes over 8-wide column vectors (VW = 8) or
// single columns.  Two passes over the row (sum of squares, then output): the
// row is re-read from cache.
template <typename TY, typename TZ, typename TO, int VW>
__global__ __launch_bounds__(256) void mamba2_gated_norm_kernel(M2NormParams p) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)p.nb * p.L) return;  // whole waves exit together
    const int b = (int)(row / p.L), l = (int)(row % p.L);
    const TY* y = static_cast<const TY*>(p.y) + (int64_t)b * p.y_sb + (int64_t)l * p.y_sl;
    const TZ* z = static_cast<const TZ*>(p.z) + (int64_t)b * p.z_sb + (int64_t)l * p.z_sl;
    TO* out = static_cast<TO*>(p.out) + (int64_t)b * p.out_sb + (int64_t)l * p.out_sl;
    auto load = [&](int c, float* yv, float* zv) {
        if constexpr (VW == 8) {
            m2_ld8(y + c, yv);
            m2_ld8(z + c, zv);
        } else {
            yv[0] = m2_ld1(y + c);
            zv[0] = m2_ld1(z + c);
        }
    };
    float ss = 0.f;
    for (int c = lane * VW; c < p.W; c += 64 * VW) {
        float yv[VW], zv[VW];
        load(c, yv, zv);
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            const float g = p.before ? yv[e] : yv[e] * m2_silu(zv[e]);
            ss += g * g;
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.f / sqrtf(ss / (float)p.W + p.eps);
    for (int c = lane * VW; c < p.W; c += 64 * VW) {
        float yv[VW], zv[VW], o[VW];
        load(c, yv, zv);
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            const float sz = m2_silu(zv[e]);
            const float g = p.before ? yv[e] : yv[e] * sz;
            o[e] = (g * inv) * p.gamma[c + e];
            if (p.before) o[e] *= sz;
        }
        if constexpr (VW == 8) {
            m2_st8(out + c, o);
        } else {
            m2_st1(out + c, o[0]);
        }
    }
}

// bf16 y and z with the whole row held in registers (packed, 8 per uint4):
// every load of a row is issued before its reduction, and the output pass
// reads nothing from memory again but gamma.  One wave per row (a wave that
// finishes frees its slot for a new row at once; a grid-stride walk over rows
// with gamma in LDS measured slower).  NI = vectors of 8 per lane, the row
// width is at most 512 NI.
__device__ __forceinline__ void m2_unpack8(const uint4 u, float* o) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o[2 * k] = __uint_as_float(w[k] << 16);
        o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}

template <typename TO, int NI>
__global__ __launch_bounds__(256) void mamba2_gated_norm_res_kernel(M2NormParams p) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)p.nb * p.L) return;  // whole waves exit together
    const int b = (int)(row / p.L), l = (int)(row % p.L);
    const bf16_t* y = static_cast<const bf16_t*>(p.y) + (int64_t)b * p.y_sb + (int64_t)l * p.y_sl;
    const bf16_t* z = static_cast<const bf16_t*>(p.z) + (int64_t)b * p.z_sb + (int64_t)l * p.z_sl;
    TO* out = static_cast<TO*>(p.out) + (int64_t)b * p.out_sb + (int64_t)l * p.out_sl;
    uint4 yr[NI], zr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int c = (i * 64 + lane) * 8;
        if (c < p.W) {
            yr[i] = *(const uint4*)(y + c);
            zr[i] = *(const uint4*)(z + c);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int c = (i * 64 + lane) * 8;
        if (c < p.W) {
            float yv[8], zv[8];
            m2_unpack8(yr[i], yv);
            m2_unpack8(zr[i], zv);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float g = p.before ? yv[e] : yv[e] * m2_silu(zv[e]);
                ss += g * g;
            }
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.f / sqrtf(ss / (float)p.W + p.eps);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int c = (i * 64 + lane) * 8;
        if (c < p.W) {
            float yv[8], zv[8], gm[8], o[8];
            m2_unpack8(yr[i], yv);
            m2_unpack8(zr[i], zv);
            m2_ld8(p.gamma + c, gm);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float sz = m2_silu(zv[e]);
                const float g = p.before ? yv[e] : yv[e] * sz;
                o[e] = (g * inv) * gm[e];
                if (p.before) o[e] *= sz;
            }
            m2_st8(out + c, o);
        }
    }
}

static bool aligned16(const void* q) { return ((uintptr_t)q & 15u) == 0; }

}  // namespace mamba

using namespace mamba;

extern "C" int mamba2_conv_fwd(const mamba2_conv_args* a, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->channels > 0 && a->nheads >= 0,
                    "batch, seqlen and channels must be >= 1, nheads >= 0");
    MAMBA_CHECK_ARG(a->kernel >= 1 && a->kernel <= kM2MaxK, "kernel must be in [1, 8]");
    MAMBA_CHECK_ARG(a->proj && a->conv_w && a->conv_state && a->xbc, "proj, conv_w, conv_state and xbc are required");
    MAMBA_CHECK_ARG(a->nheads == 0 || (a->dt_bias && a->dt), "dt_bias and dt are required when nheads > 0");
    MAMBA_CHECK_ARG((a->in_dtype == MAMBA_F32 || a->in_dtype == MAMBA_BF16) &&
                        (a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16),
                    "bad dtype");
    MAMBA_CHECK_ARG(a->xbc_offset >= 0 && a->dt_offset >= 0 && a->proj_sl >= a->xbc_offset + a->channels &&
                        a->proj_sl >= a->dt_offset + a->nheads,
                    "proj row too short for the xBC and dt slices");
    MAMBA_CHECK_ARG(a->xbc_sl >= a->channels, "xbc row stride too small");
    M2ConvParams p;
    p.nb = a->batch; p.L = a->seqlen; p.V = a->channels; p.K = a->kernel; p.H = a->nheads;
    p.proj = a->proj; p.proj_sb = a->proj_sb; p.proj_sl = a->proj_sl;
    p.xbc_off = a->xbc_offset; p.dt_off = a->dt_offset;
    p.w = a->conv_w; p.bias = a->conv_b; p.state = a->conv_state;
    p.dt_bias = a->dt_bias; p.dt_lo = a->dt_min; p.dt_hi = a->dt_max;
    p.out = a->xbc; p.out_sb = a->xbc_sb; p.out_sl = a->xbc_sl; p.dt = a->dt;
    const bool in_bf = a->in_dtype == MAMBA_BF16, out_bf = a->out_dtype == MAMBA_BF16;
    // 8-wide vectors when every row and slice is 16-byte aligned for both dtypes
    const bool vec = p.V % 8 == 0 && p.xbc_off % 8 == 0 && p.proj_sl % 8 == 0 &&
                     (p.nb == 1 || p.proj_sb % 8 == 0) && p.out_sl % 8 == 0 && (p.nb == 1 || p.out_sb % 8 == 0) &&
                     aligned16(p.proj) && aligned16(p.out);
    const int vw = vec ? 8 : 1;
    const int tiles = (p.L + kM2ConvTile - 1) / kM2ConvTile;
    const int cblocks = (p.V / vw + 255) / 256;
    MAMBA_CHECK_ARG(tiles < (1 << 30) && p.nb <= 65535, "too many tiles or batch rows");
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(tiles, cblocks, p.nb), block(256);
#define M2CONV(TI, TO, VW, KK) hipLaunchKernelGGL((mamba2_conv_kernel<TI, TO, VW, KK>), grid, block, 0, s, p)
#define M2CONV_K(TI, TO, VW)                                      \
    switch (p.K) {                                                \
        case 1: M2CONV(TI, TO, VW, 1); break;                     \
        case 2: M2CONV(TI, TO, VW, 2); break;                     \
        case 3: M2CONV(TI, TO, VW, 3); break;                     \
        case 4: M2CONV(TI, TO, VW, 4); break;                     \
        case 5: M2CONV(TI, TO, VW, 5); break;                     \
        case 6: M2CONV(TI, TO, VW, 6); break;                     \
        case 7: M2CONV(TI, TO, VW, 7); break;                     \
        default: M2CONV(TI, TO, VW, 8); break;                    \
    }
#define M2CONV_V(TI, TO) \
    if (vec) {           \
        M2CONV_K(TI, TO, 8) \
    } else {             \
        M2CONV_K(TI, TO, 1) \
    }
    if (in_bf && out_bf) {
        M2CONV_V(bf16_t, bf16_t)
    } else if (in_bf) {
        M2CONV_V(bf16_t, float)
    } else if (out_bf) {
        M2CONV_V(float, bf16_t)
    } else {
        M2CONV_V(float, float)
    }
#undef M2CONV_V
#undef M2CONV_K
#undef M2CONV
    MAMBA_CHECK_LAUNCH();
    const int64_t n = (int64_t)p.nb * p.V;
    if (in_bf)
        hipLaunchKernelGGL(mamba2_conv_state_kernel<bf16_t>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(mamba2_conv_state_kernel<float>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

extern "C" int mamba2_gated_rmsnorm(const mamba2_gated_norm_args* a, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->width > 0, "sizes must be >= 1");
    MAMBA_CHECK_ARG(a->y && a->z && a->gamma && a->out, "y, z, gamma and out are required");
    MAMBA_CHECK_ARG((a->y_dtype == MAMBA_F32 || a->y_dtype == MAMBA_BF16) &&
                        (a->z_dtype == MAMBA_F32 || a->z_dtype == MAMBA_BF16) &&
                        (a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16),
                    "bad dtype");
    MAMBA_CHECK_ARG(a->eps > 0.f, "eps must be > 0");
    M2NormParams p;
    p.nb = a->batch; p.L = a->seqlen; p.W = a->width; p.before = a->norm_before_gate != 0; p.eps = a->eps;
    p.y = a->y; p.y_sb = a->y_sb; p.y_sl = a->y_sl;
    p.z = a->z; p.z_sb = a->z_sb; p.z_sl = a->z_sl;
    p.gamma = a->gamma;
    p.out = a->out; p.out_sb = a->out_sb; p.out_sl = a->out_sl;
    const int64_t rows = (int64_t)p.nb * p.L;
    MAMBA_CHECK_ARG((rows + 3) / 4 < (1ll << 31), "too many rows");
    auto rows_ok = [&](const void* q, int64_t sb, int64_t sl) {
        return aligned16(q) && sl % 8 == 0 && (p.nb == 1 || sb % 8 == 0);
    };
    const bool vec = p.W % 8 == 0 && rows_ok(p.y, p.y_sb, p.y_sl) && rows_ok(p.z, p.z_sb, p.z_sl) &&
                     rows_ok(p.out, p.out_sb, p.out_sl) && aligned16(p.gamma);
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    const bool yb = a->y_dtype == MAMBA_BF16, zb = a->z_dtype == MAMBA_BF16, ob = a->out_dtype == MAMBA_BF16;
    if (vec && yb && zb && p.W <= 512 * 16) {
        // rows held in registers: ceil(W / 512) vectors of 8 per lane, rounded up to even
        const int ni = ((p.W + 1023) / 1024) * 2;
#define M2R1(TO, NI) \
    case NI: hipLaunchKernelGGL((mamba2_gated_norm_res_kernel<TO, NI>), grid, block, 0, s, p); break;
#define M2R(TO)                                                                            \
    switch (ni) {                                                                          \
        M2R1(TO, 2) M2R1(TO, 4) M2R1(TO, 6) M2R1(TO, 8) M2R1(TO, 10) M2R1(TO, 12) M2R1(TO, 14) \
        default: hipLaunchKernelGGL((mamba2_gated_norm_res_kernel<TO, 16>), grid, block, 0, s, p); \
    }
        if (ob) {
            M2R(bf16_t)
        } else {
            M2R(float)
        }
#undef M2R
#undef M2R1
        MAMBA_CHECK_LAUNCH();
        return MAMBA_OK;
    }
#define M2N(TY, TZ, TO)                                                                     \
    if (vec)                                                                                  \
        hipLaunchKernelGGL((mamba2_gated_norm_kernel<TY, TZ, TO, 8>), grid, block, 0, s, p); \
    else                                                                                      \
        hipLaunchKernelGGL((mamba2_gated_norm_kernel<TY, TZ, TO, 1>), grid, block, 0, s, p);
    if (yb && zb && ob) { M2N(bf16_t, bf16_t, bf16_t) }
    else if (yb && zb) { M2N(bf16_t, bf16_t, float) }
    else if (yb && ob) { M2N(bf16_t, float, bf16_t) }
    else if (yb) { M2N(bf16_t, float, float) }
    else if (zb && ob) { M2N(float, bf16_t, bf16_t) }
    else if (zb) { M2N(float, bf16_t, float) }
    else if (ob) { M2N(float, float, bf16_t) }
    else { M2N(float, float, float) }
#undef M2N
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}
