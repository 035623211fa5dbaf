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
#include <type_traits>

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
// softplus(x) = log1p(exp(x)), x itself above 20 (where the two agree in f32).
// log1p through the hardware log with Goldberg's correction, log(u) e / (u - 1)
// for u = 1 + e (a few ulp for every e > 0, no cancellation for small e): the
// library log1pf is a long polynomial sequence, and the scan's tile applies
// softplus to every (token, channel)
__device__ __forceinline__ float m1_softplus(float x) {
    if (x > 20.f) return x;
    const float e = __expf(x);
    const float u = 1.f + e;
    return u == 1.f ? e : __logf(u) * (e * __builtin_amdgcn_rcpf(u - 1.f));
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

// ---------------------------------------------------------------------------
// Time-major path for dstate 16 (u, delta, z and y contiguous along time, rows
// 16-byte aligned): 64 channels x 32-token tiles, 4 lanes per channel holding 4
// states each, as above.  A tile spans whole 128-byte lines of every row it
// touches, so each line is read from HBM once (16-token tiles read half lines
// and HBM fetched many lines twice) and y is written in whole lines.
//  * u and delta arrive by direct-to-LDS loads, 8 whole 128-byte row pieces
//    per instruction (8 lanes per line, so the memory requests are whole
//    lines), double-buffered (tile k+1 streams in while tile k is scanned),
//    with no staging registers.  Rows are [channel][32 tokens] with the eight
//    16-byte pieces of row c swizzled (piece k in slot k ^ (c % 8)): a lane
//    loads the piece its slot holds, and the scan's float4 reads of one piece
//    across 16 channels then spread over the banks.  Each wave loads the rows
//    of its own 16 channels.
//  * B and C (16 x 32 per tile) are transposed through registers into [t][n].
//  * z is prefetched into registers in the store mapping (8 tokens of one row
//    per thread, two 16-byte pieces).
//  * The scan writes y + D u over u in place; after a barrier the epilogue
//    multiplies by silu(z) and stores.
// Per tile one barrier, for the B/C tiles the waves share; everything else a
// wave touches belongs to its own 16 channels.
constexpr int kTm16Tile = 32;

template <bool GATE>
__global__ __launch_bounds__(256, 3) void mamba1_scan_tm16(Mamba1Params p) {
    constexpr int N = 16, CPB = 64, TT = kTm16Tile, NQ = TT / 4;
    __shared__ __align__(16) float s_u[2][CPB][TT];  // u, then y + D u in place (swizzled pieces)
    __shared__ __align__(16) float s_d[2][CPB][TT];  // delta (softplus'd in place)
    __shared__ __align__(16) float s_B[2][TT][N];
    __shared__ __align__(16) float s_C[2][TT][N];

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int nblk_d = (p.D + CPB - 1) / CPB;
    const int b = blockIdx.x / nblk_d, d0 = (blockIdx.x % nblk_d) * CPB;
    // scan mapping: channel c, states 4 ng .. 4 ng + 3
    const int c = tid >> 2, ng = tid & 3, d = d0 + c;
    const bool dvalid = d < p.D;
    float A2[4], h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int n = 4 * ng + k;
        A2[k] = dvalid ? p.A[(int64_t)d * p.A_sd + (int64_t)n * p.A_sn] * kLog2eM1 : 0.f;
        h[k] = (dvalid && p.h0) ? p.h0[((int64_t)b * p.D + d) * N + n] : 0.f;
    }
    const float Dd = (p.Dv && dvalid) ? p.Dv[d] : 0.f;
    const int ntile = (p.L + TT - 1) / TT;
    // byte extents of the batch row's u / delta / z / y (u's strides for all);
    // lanes with nothing to move get an offset past the end (loads read zero,
    // stores are dropped)
    const uint32_t row_bytes = (uint32_t)((((int64_t)p.D - 1) * p.u_sd + p.L) * 4);
    constexpr uint32_t kOut = 0x80000000u;
    const u32x4_t ru = buf_words(p.u + (int64_t)b * p.u_sb, row_bytes);
    const u32x4_t rd = buf_words(p.dl + (int64_t)b * p.dl_sb, row_bytes);
    const __amdgpu_buffer_rsrc_t rz = buf_rsrc(GATE ? p.z + (int64_t)b * p.z_sb : p.u, row_bytes);
    const __amdgpu_buffer_rsrc_t ry = buf_rsrc(p.y + (int64_t)b * p.y_sb, row_bytes);
    // 16-byte piece q of row r sits at float offset 4 (q ^ (r % 8)) of the row
    auto slot = [](int r, int q) { return 4 * (q ^ (r & 7)); };
    // a byte offset, or kOut where `ok` fails, as a plain select: kept opaque
    // so that the compiler neither branches around the access nor duplicates
    // it (each access below is one instruction on every path)
    auto sel = [](bool ok, uint32_t off) {
        uint32_t r = ok ? off : kOut;
        asm volatile("" : "+v"(r));
        return r;
    };
    const uint32_t sd = (uint32_t)p.u_sd;
    // DMA mapping: wave w moves rows 16 w .. 16 w + 15 (its own channels) in
    // two instructions of 8 rows; lane i -> row + i / 8, slot i % 8
    auto dma_tile = [&](int tk, int buf) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int r0 = 16 * wave + 8 * k, r = r0 + (lane >> 3);
            const int piece = (lane & 7) ^ (r & 7), t = tk * TT + 4 * piece;
            const uint32_t off = sel(d0 + r < p.D && t < p.L, ((uint32_t)(d0 + r) * sd + (uint32_t)t) * 4u);
            dma16(ru, (uint32_t)(uintptr_t)&s_u[buf][r0][0], off, 0u);
            dma16(rd, (uint32_t)(uintptr_t)&s_d[buf][r0][0], off, 0u);
        }
    };
    // B/C mapping: thread -> state tid / 16, tokens 2 (tid % 16) + {0, 1}
    const int bn = tid >> 4, bt = (tid & 15) * 2;
    const uint32_t bc_bytes = (uint32_t)(((int64_t)(N - 1) * p.B_sn + ((int64_t)p.L - 1) * p.B_sl + 1) * 4);
    const uint32_t cc_bytes = (uint32_t)(((int64_t)(N - 1) * p.C_sn + ((int64_t)p.L - 1) * p.C_sl + 1) * 4);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(p.Bm + (int64_t)b * p.B_sb, bc_bytes);
    const __amdgpu_buffer_rsrc_t rc = buf_rsrc(p.Cm + (int64_t)b * p.C_sb, cc_bytes);
    float rB[2], rC[2];
    // every load and store below is issued unconditionally (past-the-end
    // offsets read zero / drop), so that the compiler's counts of outstanding
    // memory operations are exact at the top of each tile
    auto load_bc = [&](int tk) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = tk * TT + bt + e;
            rB[e] = buf_ld4(rb, sel(t < p.L, ((uint32_t)bn * (uint32_t)p.B_sn + (uint32_t)t * (uint32_t)p.B_sl) * 4u));
            rC[e] = buf_ld4(rc, sel(t < p.L, ((uint32_t)bn * (uint32_t)p.C_sn + (uint32_t)t * (uint32_t)p.C_sl) * 4u));
        }
    };
    // store mapping: thread -> channel tid / 4, tokens 8 (tid % 4) .. + 7
    const int ec = tid >> 2, et = (tid & 3) * 8;
    const bool evalid = d0 + ec < p.D;
    // the in-place softplus touches channel tid / 4 only (8 elements per thread)
    const float sbias = (p.dbias && evalid) ? p.dbias[d0 + ec] : 0.f;
    uint4 rzv[2];
    auto eoff = [&](int tk, int k) {
        const int t = tk * TT + et + 4 * k;
        return sel(evalid && t < p.L, ((uint32_t)(d0 + ec) * sd + (uint32_t)t) * 4u);
    };
    auto load_z = [&](int tk) {
        if (GATE) {
#pragma unroll
            for (int k = 0; k < 2; ++k) rzv[k] = buf_ld16(rz, eoff(tk, k));
        }
    };

    auto tile = [&](int tk, auto partial_tag) __attribute__((always_inline)) {
        constexpr bool partial = decltype(partial_tag)::value;
        const int buf = tk & 1, t0 = tk * TT;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            s_B[buf][bt + e][bn] = rB[e];
            s_C[buf][bt + e][bn] = rC[e];
        }
        // this wave's direct-to-LDS loads of the tile: at most the previous
        // tile's two stores and this tile's two z loads were issued after them
        // (tile 0's were waited for before the first tile).  u, delta and the
        // outputs of a channel are touched by its own wave only (DMA rows,
        // scan lanes and store threads of wave w are channels 16 w .. 16 w +
        // 15), so the one barrier per tile is for B/C: every wave's writes of
        // this tile's B/C are visible, and every wave is done with the buffer
        // the next tile's B/C will overwrite
        // The count is exact only while no other vector-memory operation sits
        // between them: a register spill (scratch access) would break it, and
        // the build refuses a build of this kernel with scratch.
        constexpr int kStoresPerTile = 2;          // the epilogue's two 16-byte stores
        constexpr int kZLoadsPerTile = GATE ? 2 : 0;  // load_z
        constexpr int kAfterDma = kStoresPerTile + kZLoadsPerTile;
        static_assert(kAfterDma < 16, "vmcnt immediate is 4 bits (low field)");
        // s_waitcnt: vmcnt in bits 3:0, expcnt(7) bits 6:4, lgkmcnt(15) bits 11:8
        __builtin_amdgcn_s_waitcnt(0xF70 | kAfterDma);
        __syncthreads();
        load_bc(tk + 1);
        if (tk + 1 < ntile) dma_tile(tk + 1, buf ^ 1);
        if (p.dbias || p.softplus) {
            // delta <- softplus(delta + bias), in place
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float* v = &s_d[buf][ec][slot(ec, (et >> 2) + k)];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = p.softplus ? m1_softplus(v[e] + sbias) : v[e] + sbias;
            }
        }
        // ---- the recurrence, 4 tokens per LDS read of delta and u
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const float4 dv4 = *(const float4*)&s_d[buf][c][slot(c, q)];
            const float4 uv4 = *(const float4*)&s_u[buf][c][slot(c, q)];
            float4 bq[4], cq[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                bq[g] = *(const float4*)&s_B[buf][4 * q + g][4 * ng];
                cq[g] = *(const float4*)&s_C[buf][4 * q + g][4 * ng];
            }
            float dv[4] = {dv4.x, dv4.y, dv4.z, dv4.w}, uv[4] = {uv4.x, uv4.y, uv4.z, uv4.w};
            if (partial) {
                // past the end: identity steps (the loaded values are another
                // row's or zero), outputs not stored
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const bool ok = t0 + 4 * q + g < p.L;
                    dv[g] = ok ? dv[g] : 0.f;
                    uv[g] = ok ? uv[g] : 0.f;
                }
            }
            float yq[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float du = dv[g] * uv[g];
                const float a0 = __builtin_amdgcn_exp2f(dv[g] * A2[0]);
                const float a1 = __builtin_amdgcn_exp2f(dv[g] * A2[1]);
                const float a2 = __builtin_amdgcn_exp2f(dv[g] * A2[2]);
                const float a3 = __builtin_amdgcn_exp2f(dv[g] * A2[3]);
                h[0] = __builtin_fmaf(h[0], a0, du * bq[g].x);
                h[1] = __builtin_fmaf(h[1], a1, du * bq[g].y);
                h[2] = __builtin_fmaf(h[2], a2, du * bq[g].z);
                h[3] = __builtin_fmaf(h[3], a3, du * bq[g].w);
                yq[g] = __builtin_fmaf(cq[g].w, h[3], __builtin_fmaf(cq[g].z, h[2], __builtin_fmaf(cq[g].y, h[1], cq[g].x * h[0])));
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) yq[g] = quad_sum(yq[g]);
            // every lane of the channel holds the sums: y + D u over u
            *(float4*)&s_u[buf][c][slot(c, q)] = make_float4(__builtin_fmaf(Dd, uv[0], yq[0]), __builtin_fmaf(Dd, uv[1], yq[1]),
                                                             __builtin_fmaf(Dd, uv[2], yq[2]), __builtin_fmaf(Dd, uv[3], yq[3]));
        }
        // ---- epilogue: y = (y + D u) silu(z), two 16-byte stores per thread
        // (the wave's own rows: its LDS accesses complete in program order)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            float4 o = *(const float4*)&s_u[buf][ec][slot(ec, (et >> 2) + k)];
            if (GATE) {
                const uint4 zw = rzv[k];
                const float zv[4] = {__uint_as_float(zw.x), __uint_as_float(zw.y), __uint_as_float(zw.z),
                                     __uint_as_float(zw.w)};
                float* ov = &o.x;
#pragma unroll
                for (int e = 0; e < 4; ++e) ov[e] *= zv[e] * __builtin_amdgcn_rcpf(1.f + __expf(-zv[e]));
            }
            const uint32_t off = eoff(tk, k);
            if (partial) {
                // a piece may straddle the end: element by element
                const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = off != kOut && t0 + et + 4 * k + e < p.L;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ov[e]), ry, sel(ok, off + 4 * e), 0, 0);
                }
            } else {
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(decltype(__builtin_amdgcn_raw_buffer_load_b128(ry, 0, 0, 0)), o), ry, off, 0, 0);
            }
        }
        load_z(tk + 1);
    };

    load_bc(0);
    dma_tile(0, 0);
    load_z(0);
    __builtin_amdgcn_s_waitcnt(0);
    const int nfull = p.L / TT;
    for (int tk = 0; tk < nfull; ++tk) tile(tk, std::false_type{});
    if (nfull < ntile) tile(nfull, std::true_type{});
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

// the time-major tile path: dstate 16, time-contiguous rows at 16-byte
// aligned addresses, byte offsets inside a batch row below 2^31
static bool tm16_ok(const Mamba1Params& p) {
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    return p.N == 16 && p.u_sl == 1 && p.u_sd % 4 == 0 && p.u_sd >= p.L && al16(p.u) && al16(p.dl) &&
           al16(p.y) && (!p.z || al16(p.z)) && p.u_sb % 4 == 0 && p.dl_sb % 4 == 0 && p.y_sb % 4 == 0 &&
           (!p.z || p.z_sb % 4 == 0) && (((int64_t)p.D - 1) * p.u_sd + p.L) * 4 < (1ll << 31) &&
           p.B_sn >= 0 && p.B_sl >= 0 && p.C_sn >= 0 && p.C_sl >= 0 &&
           ((int64_t)(p.N - 1) * p.B_sn + ((int64_t)p.L - 1) * p.B_sl + 1) * 4 < (1ll << 31) &&
           ((int64_t)(p.N - 1) * p.C_sn + ((int64_t)p.L - 1) * p.C_sl + 1) * 4 < (1ll << 31);
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
    int nfast = (same_strides && fits32) ? p.N : 0;
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    if (nfast == 16 && tm16_ok(p)) {
        const int nblk = p.nb * ((p.D + 63) / 64);
        if (p.z)
            hipLaunchKernelGGL((mamba1_scan_tm16<true>), dim3(nblk), dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((mamba1_scan_tm16<false>), dim3(nblk), dim3(256), 0, stream, p);
        nfast = -1;
    }
    switch (nfast) {
        case -1: break;
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
