// Mamba-3 single-pass SSD forward, gfx950 MFMA path (bf16 v/B/C/y, f32 state),
// headdim 64, dstate 128, MIMO rank M dividing 32.
//
// Reference: Mamba3SingleSsdBackendExt::single_ssd_serial_recalculated
// (src/mamba3/single_ssd/ssd/serial_recalculated/serial_recalculated.rs:86-291).
//
// The MIMO rank is fused into the time axis (position f = M t + m, the
// reference's fused L*M index, single_ssd/ssd/minimal.rs:152-172): with v, B,
// C and y laid out [.., l, m, ..] that axis is a single stride.  One workgroup
// (4 waves) per (batch, head, 32-wide half of headdim) walks fused chunks of
// QF = 128 positions (QF / M time steps) in order with the state in MFMA
// accumulators (K4 never touches HBM).  B and C are per head here, so unlike
// the Mamba-2 path there is no shared C.B^T workspace: each 32 x 32 tile of
// the chunk's C.B^T is computed on the fly, as D'[j][i] = B_j . C_i on
// v_mfma_f32_32x32x16_bf16 (A = B rows, B operand = C rows, both row-major in
// LDS).  Its accumulator layout (lane = column i, rows j = 8(v/4) + 4 half +
// v%4) is used directly as the B operand of y^T[p][i] += sum_j v^T[p][j]
// M[j][i]: the k order is permuted, and the v^T fragments are read with the
// same permutation (two 8-byte LDS reads), which leaves the product unchanged.
// For output tile it (r0 = 32 it), with e_i = exp(cs_i - cs_r0) <= 1:
//   y_i = e_i [ exp(cs_r0) C_i.h_in + sum_{j < r0} (B_j.C_i) f_it[j] v_j ]
//         + sum_{r0 <= j < 32 it + 32} (B_j.C_i) k(j, i) v_j
// with f_it[j] = scale_j exp(cs_r0 - cs_j) tabulated per chunk, and on the
// diagonal tile k(j, i) = scale_j exp(cs_i - cs_j) for step(j) < step(i),
// gamma_step(i) for step(j) == step(i), 0 otherwise.  The chunk state uses
// w_j = scale_j exp(cs_end - cs_j) applied to a transposed copy of B in LDS.
#include <cstdlib>

#include "common.h"

namespace mamba {

struct Ssd3MfmaParams {
    int nb, L, M, H, G, nch;  // L = fused length (seqlen * M); nch fused chunks of QF
    const bf16_t* v; int64_t v_sb, v_sf, v_sh;  // fused stride v_sf = v_sm
    const float* da; int64_t da_sb, da_sl, da_sh;
    const float* gm; int64_t gm_sb, gm_sl, gm_sh;
    const float* sc; int64_t sc_sb, sc_sl, sc_sh;
    const bf16_t* Bm; int64_t B_sb, B_sf, B_sg;
    const bf16_t* Cm; int64_t C_sb, C_sf, C_sg;
    const float* h0;
    bf16_t* y; int64_t y_sb, y_sf, y_sh;
    float* hT;
};

typedef __bf16 s3_bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 s3_bf16x4_t __attribute__((ext_vector_type(4)));
typedef float s3_f32x16_t __attribute__((ext_vector_type(16)));

constexpr float kLog2eS3 = 1.4426950408889634f;

__device__ __forceinline__ s3_f32x16_t s3_mfma(s3_bf16x8_t a, s3_bf16x8_t b, s3_f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ s3_f32x16_t s3_zero() {
    s3_f32x16_t z;
#pragma unroll
    for (int v = 0; v < 16; ++v) z[v] = 0.f;
    return z;
}

__device__ __forceinline__ uint4 s3_ld16(const void* ptr, bool ok) {
    return ok ? *(const uint4*)ptr : make_uint4(0u, 0u, 0u, 0u);
}

__device__ __forceinline__ float s3_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float s3_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int QF>
__global__ __launch_bounds__(256, 1) void ssd3_scan_mfma(Ssd3MfmaParams p) {
    constexpr int N = 128;
    constexpr int T = QF / 32;            // i-tiles per chunk (one per wave)
    static_assert(T == 4, "one output tile per wave");
    constexpr int XP = QF + 8;            // s_xT / s_BT row pitch (bf16)
    constexpr int RP = N + 8;             // s_B / s_C / s_h row pitch (bf16)
    constexpr int NK = N / 16;            // k-steps over dstate
    constexpr int KS = QF / 16;           // k-steps over the chunk
    constexpr int XI = (QF / 2) * 4;      // v staging items: (row pair, 8-wide headdim chunk)
    constexpr int BI = (QF / 2) * (N / 8);  // B staging items: (row pair, 8-wide dstate chunk)
    constexpr int CI = QF * (N / 8);        // C staging items: (row, 8-wide dstate chunk)
    constexpr int XPT = (XI + 255) / 256, BPT = BI / 256, CPT = CI / 256;
    __shared__ __align__(16) bf16_t s_xT[32][XP];
    __shared__ __align__(16) bf16_t s_B[QF][RP];
    __shared__ __align__(16) bf16_t s_C[QF][RP];
    __shared__ __align__(16) bf16_t s_BT[N][XP];
    __shared__ __align__(16) bf16_t s_h[32][RP];
    __shared__ __align__(16) bf16_t s_y[4][32][40];
    __shared__ __align__(16) float s_cs2[QF];
    __shared__ __align__(16) float s_sc[QF];
    __shared__ __align__(16) float s_gm[QF];
    __shared__ __align__(16) float s_w[QF];
    __shared__ __align__(16) float s_f[T - 1][QF];
    __shared__ float s_red[4];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, half = lane >> 5;
    // XCD-aware mapping: the two headdim halves of a head (sharing B/C) and
    // neighbouring heads of a batch row land on one XCD
    const int nwg = p.nb * p.H * 2;
    int w = blockIdx.x;
    if ((nwg & 7) == 0) w = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    const int ph = w & 1, h = (w >> 1) % p.H, b = (w >> 1) / p.H;
    const int g = h / (p.H / p.G);
    const int p0 = ph * 32;
    const int lgM = __builtin_ctz(p.M);  // the MIMO rank is a power of two dividing 32

    // state tile of this wave: headdim rows p0..p0+31, dstate columns 32 wave..
    s3_f32x16_t hacc;
    const int64_t hbase = ((int64_t)b * p.H + h) * 64 * N;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int pp = p0 + 8 * (v >> 2) + 4 * half + (v & 3);
        hacc[v] = p.h0 ? p.h0[hbase + pp * N + wave * 32 + r] : 0.f;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v)
        s_h[8 * (v >> 2) + 4 * half + (v & 3)][wave * 32 + r] = __builtin_bit_cast(bf16_t, (__bf16)hacc[v]);

    const bf16_t* vhead = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + p0;
    const bf16_t* bhead = p.Bm + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    const bf16_t* chead = p.Cm + (int64_t)b * p.C_sb + (int64_t)g * p.C_sg;
    bf16_t* yhead = p.y + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh + p0;

    // ---- register prefetch of one chunk
    uint4 xq[XPT][2], bq[BPT][2], cq[CPT];
    float daq = 0.f, scq = 0.f, gmq = 0.f;
    auto fetch = [&](int c) {
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            const int fp = item >> 2, pv = item & 3;
            const int f0 = c * QF + 2 * fp;
            const bool ok = item < XI;
            xq[k][0] = s3_ld16(vhead + (int64_t)f0 * p.v_sf + pv * 8, ok && f0 < p.L);
            xq[k][1] = s3_ld16(vhead + (int64_t)(f0 + 1) * p.v_sf + pv * 8, ok && f0 + 1 < p.L);
        }
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            const int fp = item >> 4, nv = item & 15;
            const int f0 = c * QF + 2 * fp;
            bq[k][0] = s3_ld16(bhead + (int64_t)f0 * p.B_sf + nv * 8, f0 < p.L);
            bq[k][1] = s3_ld16(bhead + (int64_t)(f0 + 1) * p.B_sf + nv * 8, f0 + 1 < p.L);
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            const int f = c * QF + (item >> 4), nv = item & 15;
            cq[k] = s3_ld16(chead + (int64_t)f * p.C_sf + nv * 8, f < p.L);
        }
        daq = scq = gmq = 0.f;
        const int f = c * QF + threadIdx.x;
        if (threadIdx.x < QF && f < p.L) {
            const int t = f >> lgM;
            if (f - (t << lgM) == 0) daq = p.da[(int64_t)b * p.da_sb + (int64_t)t * p.da_sl + (int64_t)h * p.da_sh];
            scq = p.sc[(int64_t)b * p.sc_sb + (int64_t)t * p.sc_sl + (int64_t)h * p.sc_sh];
            gmq = p.gm[(int64_t)b * p.gm_sb + (int64_t)t * p.gm_sl + (int64_t)h * p.gm_sh];
        }
    };
    fetch(0);

    for (int c = 0; c < p.nch; ++c) {
        // ---- commit v (time-major), B and C (row-major), per-position tables
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            if (item < XI) {
                const int fp = item >> 2, pv = item & 3;
                const uint32_t a0[4] = {xq[k][0].x, xq[k][0].y, xq[k][0].z, xq[k][0].w};
                const uint32_t a1[4] = {xq[k][1].x, xq[k][1].y, xq[k][1].z, xq[k][1].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    *(uint32_t*)&s_xT[pv * 8 + 2 * e][2 * fp] = (a0[e] & 0xffffu) | (a1[e] << 16);
                    *(uint32_t*)&s_xT[pv * 8 + 2 * e + 1][2 * fp] = (a0[e] >> 16) | (a1[e] & 0xffff0000u);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            const int fp = item >> 4, nv = item & 15;
            *(uint4*)&s_B[2 * fp][nv * 8] = bq[k][0];
            *(uint4*)&s_B[2 * fp + 1][nv * 8] = bq[k][1];
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            *(uint4*)&s_C[item >> 4][(item & 15) * 8] = cq[k];
        }
        {
            float vsum = wave_incl_scan(daq * kLog2eS3);
            if (lane == 63) s_red[wave] = vsum;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 3; ++k)
                if (k < wave) vsum += s_red[k];
            if (threadIdx.x < QF) {
                s_cs2[threadIdx.x] = vsum;
                s_sc[threadIdx.x] = scq;
                s_gm[threadIdx.x] = gmq;
            }
        }
        __syncthreads();
        const float cs2_end = s_cs2[QF - 1];
        if (threadIdx.x < QF) {
            const int j = threadIdx.x;
            const float csj = s_cs2[j];
            s_w[j] = scq * __builtin_amdgcn_exp2f(cs2_end - csj);
#pragma unroll
            for (int it = 1; it < T; ++it)
                if (j < it * 32) s_f[it - 1][j] = scq * __builtin_amdgcn_exp2f(s_cs2[it * 32] - csj);
        }
        __syncthreads();
        // w-scaled transposed B (the state GEMM's B operand): s_BT[n][j] = w_j B[j][n]
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            const int item = threadIdx.x + 256 * k;
            const int fp = item >> 4, nv = item & 15;
            const float w0 = s_w[2 * fp], w1 = s_w[2 * fp + 1];
            const uint32_t a0[4] = {bq[k][0].x, bq[k][0].y, bq[k][0].z, bq[k][0].w};
            const uint32_t a1[4] = {bq[k][1].x, bq[k][1].y, bq[k][1].z, bq[k][1].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = (uint32_t)f32_to_bf16(s3_lo(a0[e]) * w0) | ((uint32_t)f32_to_bf16(s3_lo(a1[e]) * w1) << 16);
                const uint32_t hi = (uint32_t)f32_to_bf16(s3_hi(a0[e]) * w0) | ((uint32_t)f32_to_bf16(s3_hi(a1[e]) * w1) << 16);
                *(uint32_t*)&s_BT[nv * 8 + 2 * e][2 * fp] = lo;
                *(uint32_t*)&s_BT[nv * 8 + 2 * e + 1][2 * fp] = hi;
            }
        }

        // ---- y for output tile it = wave
        {
            const int it = wave;
            const int il = it * 32 + r;  // this lane's output position (B-operand column)
            s3_bf16x8_t cfr[NK];
#pragma unroll
            for (int kn = 0; kn < NK; ++kn) cfr[kn] = *(const s3_bf16x8_t*)&s_C[il][kn * 16 + 8 * half];
            const float cs2_i = s_cs2[il], cs2_r0 = s_cs2[it * 32];
            s3_f32x16_t yacc = s3_zero();
            // inter-chunk term h_in . C_i^T
#pragma unroll
            for (int kn = 0; kn < NK; ++kn) {
                const s3_bf16x8_t a = *(const s3_bf16x8_t*)&s_h[r][kn * 16 + 8 * half];
                yacc = s3_mfma(a, cfr[kn], yacc);
            }
            {
                const float sc0 = __builtin_amdgcn_exp2f(cs2_r0);
#pragma unroll
                for (int v = 0; v < 16; ++v) yacc[v] *= sc0;
            }
            // C.B^T tile jt -> scaled bf16 B operand -> two y k-steps
            auto ytile = [&](int jt, auto factor) {
                s3_f32x16_t d = s3_zero();
#pragma unroll
                for (int kn = 0; kn < NK; ++kn) {
                    const s3_bf16x8_t a = *(const s3_bf16x8_t*)&s_B[jt * 32 + r][kn * 16 + 8 * half];
                    d = s3_mfma(a, cfr[kn], d);
                }
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    s3_bf16x8_t bop;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int v = 8 * kk + e;
                        const int j = jt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                        bop[e] = (__bf16)(d[v] * factor(j));
                    }
                    // v^T[p][j] in the same (permuted) k order: j = jt*32 + 16 kk + {0..3, 8..11} + 4 half
                    const int j0 = jt * 32 + 16 * kk + 4 * half;
                    const s3_bf16x4_t lo = *(const s3_bf16x4_t*)&s_xT[r][j0];
                    const s3_bf16x4_t hi = *(const s3_bf16x4_t*)&s_xT[r][j0 + 8];
                    s3_bf16x8_t a;
                    a[0] = lo[0]; a[1] = lo[1]; a[2] = lo[2]; a[3] = lo[3];
                    a[4] = hi[0]; a[5] = hi[1]; a[6] = hi[2]; a[7] = hi[3];
                    yacc = s3_mfma(a, bop, yacc);
                }
            };
            for (int jt = 0; jt < it; ++jt) ytile(jt, [&](int j) { return s_f[it - 1][j]; });
            {
                const float ei = __builtin_amdgcn_exp2f(cs2_i - cs2_r0);
#pragma unroll
                for (int v = 0; v < 16; ++v) yacc[v] *= ei;
            }
            const int ti = il >> lgM;  // chunks and tiles start on step boundaries
            const float gmi = s_gm[il];
            ytile(it, [&](int j) {
                const int tj = j >> lgM;
                return tj < ti ? s_sc[j] * __builtin_amdgcn_exp2f(cs2_i - s_cs2[j]) : (tj == ti ? gmi : 0.f);
            });
            // stage the 32 (p) x 32 (time) tile: lane holds y[il][p = 8(v/4) + 4 half + v%4]
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                uint2 pk;
                pk.x = (uint32_t)f32_to_bf16(yacc[4 * gq]) | ((uint32_t)f32_to_bf16(yacc[4 * gq + 1]) << 16);
                pk.y = (uint32_t)f32_to_bf16(yacc[4 * gq + 2]) | ((uint32_t)f32_to_bf16(yacc[4 * gq + 3]) << 16);
                *(uint2*)&s_y[wave][r][8 * gq + 4 * half] = pk;
            }
            __builtin_amdgcn_wave_barrier();  // LDS ops of one wave complete in order
            // 32 rows x 64 bytes: 4 lanes per row, 16 rows per instruction
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int row = q * 16 + (lane >> 2), ch = lane & 3;
                const int f = c * QF + it * 32 + row;
                if (f < p.L) *(uint4*)(yhead + (int64_t)f * p.y_sf + ch * 8) = *(const uint4*)&s_y[wave][row][ch * 8];
            }
        }
        __syncthreads();  // s_B / s_C / s_h / s_xT reads of the y phase done
        // ---- next chunk's loads land during the state GEMM
        if (c + 1 < p.nch) fetch(c + 1);
        // ---- state: h <- exp(cs_end) h + sum_j v^T[p][j] (w_j B[j][n]) for n tile = wave
        {
            const float dec = __builtin_amdgcn_exp2f(cs2_end);
#pragma unroll
            for (int v = 0; v < 16; ++v) hacc[v] *= dec;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const s3_bf16x8_t a = *(const s3_bf16x8_t*)&s_xT[r][ks * 16 + 8 * half];
                const s3_bf16x8_t bo = *(const s3_bf16x8_t*)&s_BT[wave * 32 + r][ks * 16 + 8 * half];
                hacc = s3_mfma(a, bo, hacc);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
                s_h[8 * (v >> 2) + 4 * half + (v & 3)][wave * 32 + r] = __builtin_bit_cast(bf16_t, (__bf16)hacc[v]);
        }
        __syncthreads();  // s_h / s_xT / s_BT consumed before the next commit
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int pp = p0 + 8 * (v >> 2) + 4 * half + (v & 3);
        p.hT[hbase + pp * N + wave * 32 + r] = hacc[v];
    }
}

// Fast-path conditions (the caller has validated the arguments).
bool ssd3_mfma_supported(const mamba_ssd3_args* a) {
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    return a->io_dtype == MAMBA_BF16 && a->headdim == 64 && a->dstate == 128 && 32 % a->mimo == 0 &&
           a->ngroups > 0 && a->nheads % a->ngroups == 0 &&
           a->v_sl == (int64_t)a->mimo * a->v_sm && a->y_sl == (int64_t)a->mimo * a->y_sm &&
           a->B_sl == (int64_t)a->mimo * a->B_sm && a->C_sl == (int64_t)a->mimo * a->C_sm &&
           a->v_sm % 8 == 0 && a->y_sm % 8 == 0 && a->B_sm % 8 == 0 && a->C_sm % 8 == 0 && a->v_sh % 8 == 0 &&
           a->y_sh % 8 == 0 && a->B_sg % 8 == 0 && a->C_sg % 8 == 0 && a->v_sb % 8 == 0 && a->y_sb % 8 == 0 &&
           a->B_sb % 8 == 0 && a->C_sb % 8 == 0 && al16(a->v) && al16(a->y) && al16(a->B) && al16(a->C) &&
           (int64_t)a->seqlen * a->mimo < (1ll << 30);
}

int ssd3_mfma_launch(const mamba_ssd3_args* a, hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    constexpr int QF = 128;
    Ssd3MfmaParams p;
    p.nb = a->batch; p.M = a->mimo; p.H = a->nheads; p.G = a->ngroups;
    p.L = a->seqlen * a->mimo;
    p.nch = (p.L + QF - 1) / QF;
    p.v = static_cast<const bf16_t*>(a->v); p.v_sb = a->v_sb; p.v_sf = a->v_sm; p.v_sh = a->v_sh;
    p.da = a->da; p.da_sb = a->da_sb; p.da_sl = a->da_sl; p.da_sh = a->da_sh;
    p.gm = a->gamma; p.gm_sb = a->gamma_sb; p.gm_sl = a->gamma_sl; p.gm_sh = a->gamma_sh;
    p.sc = a->scale; p.sc_sb = a->scale_sb; p.sc_sl = a->scale_sl; p.sc_sh = a->scale_sh;
    p.Bm = static_cast<const bf16_t*>(a->B); p.B_sb = a->B_sb; p.B_sf = a->B_sm; p.B_sg = a->B_sg;
    p.Cm = static_cast<const bf16_t*>(a->C); p.C_sb = a->C_sb; p.C_sf = a->C_sm; p.C_sg = a->C_sg;
    p.h0 = a->initial_state;
    p.y = static_cast<bf16_t*>(a->y); p.y_sb = a->y_sb; p.y_sf = a->y_sm; p.y_sh = a->y_sh;
    p.hT = a->final_state;
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    hipLaunchKernelGGL(ssd3_scan_mfma<QF>, dim3(p.nb * p.H * 2), dim3(256), 0, stream, p);
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    return MAMBA_OK;
}

}  // namespace mamba
