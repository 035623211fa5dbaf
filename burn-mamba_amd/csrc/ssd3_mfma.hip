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

#include "ssd3_core.h"

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

// UNIT: the double-SSD seam, scale = gamma = 1 at every position (no tables read)
// 8 waves: waves 0-3 each form one 32-position output tile, waves 4-7 each
// update one 32-column dstate tile of the state, so the two halves of the
// chunk's MFMA work run side by side on every SIMD (two waves per SIMD);
// every wave shares the staging.
template <int QF, bool UNIT>
__global__ __launch_bounds__(512, 1) void ssd3_scan_mfma(Ssd3MfmaParams p) {
    constexpr int N = 128;
    constexpr int T = QF / 32;            // output tiles per chunk (one per wave)
    static_assert(T == 4, "one output tile per wave");
    constexpr int NK = N / 16;            // k-steps over dstate
    constexpr int XI = (QF / 2) * 4;      // v staging items: (position pair, 8-wide headdim piece)
    constexpr int BI = (QF / 2) * (N / 8);  // B staging items: (position pair, 8-wide dstate piece)
    constexpr int NT = 512;               // threads
    constexpr int XPT = (XI + NT - 1) / NT, BPT = BI / NT;
    __shared__ Ssd3Lds<QF> S;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, half = lane >> 5;
    const bool st_wave = wave >= 4;       // waves 4-7: the state; 0-3: the y tiles
    const int w4 = wave & 3;              // the state wave's dstate tile / the y wave's output tile
    // XCD-aware mapping: the two headdim halves of a head (same B/C rows) and
    // neighbouring heads of a batch row land on one XCD
    const int nwg = p.nb * p.H * 2;
    int w = blockIdx.x;
    if ((nwg & 7) == 0) w = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    const int ph = w & 1, h = (w >> 1) % p.H, b = (w >> 1) / p.H;
    const int g = h / (p.H / p.G);
    const int p0 = ph * 32;
    const int lgM = __builtin_ctz(p.M);  // the MIMO rank is a power of two dividing 32

    // state tile of a state wave: headdim rows p0..p0+31, dstate columns 32 w4..
    s3_f32x16_t hacc;
    const int64_t hbase = ((int64_t)b * p.H + h) * 64 * N;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int pp = p0 + 8 * (v >> 2) + 4 * half + (v & 3);
        hacc[v] = (st_wave && p.h0) ? p.h0[hbase + pp * N + w4 * 32 + r] : 0.f;
    }
    if (st_wave) ssd3_put_state(S, hacc, 0, w4, r, half);

    const bf16_t* vhead = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + p0;
    const bf16_t* bhead = p.Bm + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    const bf16_t* chead = p.Cm + (int64_t)b * p.C_sb + (int64_t)g * p.C_sg;
    bf16_t* yhead = p.y + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh + p0;
    const float* dahead = p.da + (int64_t)b * p.da_sb + (int64_t)h * p.da_sh;
    const float* schead = p.sc + (int64_t)b * p.sc_sb + (int64_t)h * p.sc_sh;
    const float* gmhead = p.gm + (int64_t)b * p.gm_sb + (int64_t)h * p.gm_sh;

    // per-thread byte offsets within a chunk (the host bounds a chunk's span below 2^31 bytes)
    const uint32_t v_rs = (uint32_t)p.v_sf * 2, b_rs = (uint32_t)p.B_sf * 2, c_rs = (uint32_t)p.C_sf * 2;
    // v items: position pair threadIdx.x / 4 (threads 0-255), 8-wide headdim piece threadIdx.x % 4
    const uint32_t vo = (uint32_t)((threadIdx.x & 255) >> 2) * 2 * v_rs + (threadIdx.x & 3) * 16;
    // B items: position pair fp = tid / 16 (+32 per k), 8-wide dstate piece nv
    const int b_fp = threadIdx.x >> 4, b_nv = threadIdx.x & 15;
    const uint32_t bo = (uint32_t)b_fp * 2 * b_rs + b_nv * 16;
    const uint32_t co = (uint32_t)(w4 * 32 + r) * c_rs + 16 * half;
    // step of this thread's position within the chunk; threads past the chunk's
    // positions read one step past its end (zero through the buffer's extent)
    const int tpos = min((int)threadIdx.x, QF) >> lgM;
    const uint32_t dao = (uint32_t)tpos * (uint32_t)p.da_sl * 4, sco = (uint32_t)tpos * (uint32_t)p.sc_sl * 4,
                   gmo = (uint32_t)tpos * (uint32_t)p.gm_sl * 4;
    const bool first_m = (threadIdx.x & ((1 << lgM) - 1)) == 0;

    // ---- register prefetch of one chunk: v and B pieces for the LDS commit, tables
    static_assert(XPT == 1, "one v item per thread");
    uint4 xq[XPT][2], bq[BPT][2], cn[NK];
    float daq = 0.f, scq = 0.f, gmq = 0.f;
    auto fetch = [&](int c) {
        const int rows = min(QF, p.L - c * QF);  // valid positions of the chunk
        const int steps = rows >> lgM;
        const int64_t f0 = (int64_t)c * QF;
        // the v items sit in waves 0-3: the state waves' copies read nothing
        const __amdgpu_buffer_rsrc_t rv = s3_rsrc(vhead + f0 * p.v_sf, (uint32_t)(wave < 4 ? rows : 0) * v_rs);
        const __amdgpu_buffer_rsrc_t rb = s3_rsrc(bhead + f0 * p.B_sf, (uint32_t)rows * b_rs);
        xq[0][0] = s3_bld16(rv, vo);
        xq[0][1] = s3_bld16(rv, vo + v_rs);
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            bq[k][0] = s3_bld16(rb, bo + (uint32_t)k * 64 * b_rs);
            bq[k][1] = s3_bld16(rb, bo + (uint32_t)k * 64 * b_rs + b_rs);
        }
        const int64_t t0 = f0 >> lgM;
        const __amdgpu_buffer_rsrc_t rda = s3_rsrc(dahead + t0 * p.da_sl, (uint32_t)steps * (uint32_t)p.da_sl * 4);
        const float dav = s3_bld4(rda, dao);
        daq = first_m ? dav : 0.f;  // da enters the cumulative sum once per step
        if constexpr (UNIT) {
            // positions past the end carry v = B = 0, so their unit factor is inert
            scq = 1.f;
            gmq = 1.f;
        } else {
            const __amdgpu_buffer_rsrc_t rsc = s3_rsrc(schead + t0 * p.sc_sl, (uint32_t)steps * (uint32_t)p.sc_sl * 4);
            const __amdgpu_buffer_rsrc_t rgm = s3_rsrc(gmhead + t0 * p.gm_sl, (uint32_t)steps * (uint32_t)p.gm_sl * 4);
            scq = s3_bld4(rsc, sco);
            gmq = s3_bld4(rgm, gmo);
        }
    };
    // this wave's C fragments of a chunk: issued a chunk ahead, after the
    // current fragments are dead, so only one set is held in registers
    auto fetch_c = [&](int c) {
        const int rows = min(QF, p.L - c * QF);
        const __amdgpu_buffer_rsrc_t rc = s3_rsrc(chead + (int64_t)c * QF * p.C_sf, (uint32_t)rows * c_rs);
#pragma unroll
        for (int kn = 0; kn < NK; ++kn) cn[kn] = s3_bld16(rc, co + 32 * kn);
    };
    fetch(0);
    if (!st_wave) fetch_c(0);

    for (int c = 0; c < p.nch; ++c) {
        const int cur = c & 1;
        // the lane coordinates as opaque values: the per-lane LDS addresses of
        // the tiles below are loop-invariant, and hoisted out of the chunk loop
        // they would hold registers the two wave roles cannot spare
        int tid_o = (int)threadIdx.x;
        asm volatile("" : "+v"(tid_o));
        const int lane = tid_o & 63, r = lane & 31, half = lane >> 5;
        // ---- per-position tables: one block scan of da (log2 units); the
        // wave totals and the local values at tile starts go through LDS
        const float loc = wave_incl_scan(daq * kLog2eS3);
        if (lane == 63 && wave < 4) S.red[wave] = loc;
        if ((threadIdx.x & 31) == 0 && threadIdx.x < QF) S.anc[threadIdx.x >> 5] = loc;
        __syncthreads();
        const float cs_end = (S.red[0] + S.red[1]) + (S.red[2] + S.red[3]);
        if (threadIdx.x < QF) {
            const int j = threadIdx.x;
            float off = 0.f;
#pragma unroll
            for (int k = 0; k < 3; ++k)
                if (k < wave) off += S.red[k];
            const float csj = loc + off;
            S.cs2[j] = csj;
            S.st[j] = (float)(j >> lgM);
            S.sc[j] = scq;
            S.gm[j] = gmq;
            S.w[j] = scq * __builtin_amdgcn_exp2f(cs_end - csj);
#pragma unroll
            for (int it = 1; it < T; ++it) {
                if (j < it * 32) {
                    float anchor = S.anc[it];
#pragma unroll
                    for (int k = 0; k < 3; ++k)
                        if (k < (it >> 1)) anchor += S.red[k];
                    S.f[it - 1][j] = scq * __builtin_amdgcn_exp2f(anchor - csj);
                }
            }
        }
        // ---- commit B (row-major) to LDS
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            const int fp = b_fp + 32 * k;
            *(uint4*)&S.B[2 * fp][b_nv * 8] = bq[k][0];
            *(uint4*)&S.B[2 * fp + 1][b_nv * 8] = bq[k][1];
        }
        __syncthreads();  // w table ready
        // ---- commit v^T and w-scaled v^T
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int item = threadIdx.x + NT * k;
            if (item < XI) {
                const int fp = item >> 2, pv = item & 3;
                const float w0 = S.w[2 * fp], w1 = S.w[2 * fp + 1];
                const uint32_t a0[4] = {xq[k][0].x, xq[k][0].y, xq[k][0].z, xq[k][0].w};
                const uint32_t a1[4] = {xq[k][1].x, xq[k][1].y, xq[k][1].z, xq[k][1].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    *(uint32_t*)&S.xT[pv * 8 + 2 * e][2 * fp] = (a0[e] & 0xffffu) | (a1[e] << 16);
                    *(uint32_t*)&S.xT[pv * 8 + 2 * e + 1][2 * fp] = (a0[e] >> 16) | (a1[e] & 0xffff0000u);
                    const float va[4] = {s3_lo(a0[e]), s3_lo(a1[e]), s3_hi(a0[e]), s3_hi(a1[e])};
                    const float wa[4] = {w0, w1, w0, w1};
                    s3_bf16x4_t q, ql;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        __bf16 hi, lo;
                        s3_split(va[i], wa[i], hi, lo);
                        q[i] = hi;
                        ql[i] = lo;
                    }
                    const uint2 qq = __builtin_bit_cast(uint2, q), qql = __builtin_bit_cast(uint2, ql);
                    *(uint32_t*)&S.xTw[pv * 8 + 2 * e][2 * fp] = qq.x;
                    *(uint32_t*)&S.xTw[pv * 8 + 2 * e + 1][2 * fp] = qq.y;
                    *(uint32_t*)&S.xTwl[pv * 8 + 2 * e][2 * fp] = qql.x;
                    *(uint32_t*)&S.xTwl[pv * 8 + 2 * e + 1][2 * fp] = qql.y;
                }
            }
        }
        s3_bf16x8_t cfr[NK];
#pragma unroll
        for (int kn = 0; kn < NK; ++kn) cfr[kn] = __builtin_bit_cast(s3_bf16x8_t, cn[kn]);  // y waves' only
        // ---- the next chunk's loads land during this chunk's MFMA work
        if (c + 1 < p.nch) fetch(c + 1);
        __syncthreads();
        if (st_wave) {
            // ---- state: h <- exp(cs_end) h + sum_j (w_j v^T[p][j]) B[j][n], n tile = w4
            const float dec = __builtin_amdgcn_exp2f(cs_end);
#pragma unroll
            for (int v = 0; v < 16; ++v) hacc[v] *= dec;
            ssd3_state_update(S, hacc, w4, r, half);
            ssd3_put_state(S, hacc, cur ^ 1, w4, r, half);
        } else {
            // ---- y for output tile = wave
            s3_f32x16_t yacc;
            switch (wave) {
                case 0: ssd3_y_tile<QF, 0>(S, cfr, cur, r, half, yacc); break;
                case 1: ssd3_y_tile<QF, 1>(S, cfr, cur, r, half, yacc); break;
                case 2: ssd3_y_tile<QF, 2>(S, cfr, cur, r, half, yacc); break;
                default: ssd3_y_tile<QF, 3>(S, cfr, cur, r, half, yacc); break;
            }
            // stage the 32 (time) x 32 (p) tile: lane holds y[i][p = 8(v/4) + 4 half + v%4]
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const s3_bf16x4_t q = {(__bf16)yacc[4 * gq], (__bf16)yacc[4 * gq + 1], (__bf16)yacc[4 * gq + 2],
                                       (__bf16)yacc[4 * gq + 3]};
                *(s3_bf16x4_t*)&S.y[wave][r][8 * gq + 4 * half] = q;
            }
            __builtin_amdgcn_wave_barrier();  // LDS ops of one wave complete in order
            if (c + 1 < p.nch) fetch_c(c + 1);
            // 32 rows x 64 bytes: 4 lanes per row, 16 rows per instruction
            const int rows = min(QF, p.L - c * QF);
            const uint32_t y_rs = (uint32_t)p.y_sf * 2;
            const __amdgpu_buffer_rsrc_t ry = s3_rsrc(yhead + (int64_t)c * QF * p.y_sf, (uint32_t)rows * y_rs);
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int row = q * 16 + (lane >> 2), ch = lane & 3;
                const uint4 val = *(const uint4*)&S.y[wave][row][ch * 8];
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(decltype(__builtin_amdgcn_raw_buffer_load_b128(ry, 0, 0, 0)), val),
                                                       ry, (uint32_t)(wave * 32 + row) * y_rs + ch * 16, 0, 0);
            }
        }
        __syncthreads();  // LDS reads of this chunk done before the next commit
    }
    if (st_wave)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int pp = p0 + 8 * (v >> 2) + 4 * half + (v & 3);
            p.hT[hbase + pp * N + w4 * 32 + r] = hacc[v];
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
    // gamma and scale are NULL only for the double-SSD seam (unit coefficients)
    if (a->gamma == nullptr)
        hipLaunchKernelGGL((ssd3_scan_mfma<QF, true>), dim3(p.nb * p.H * 2), dim3(512), 0, stream, p);
    else
        hipLaunchKernelGGL((ssd3_scan_mfma<QF, false>), dim3(p.nb * p.H * 2), dim3(512), 0, stream, p);
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    return MAMBA_OK;
}

}  // namespace mamba
