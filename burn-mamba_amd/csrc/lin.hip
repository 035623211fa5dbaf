// Weight-streaming dense product Y[M, N] = A[M, K] W[K, N] for decode steps
// (M = batch <= 256): the in_proj / out_proj of the recurrent blocks.
//
// At decode the product is bound by streaming W from HBM (every weight byte is
// used M times, M small), so the design point is "each weight byte read once,
// in whole 1 KB wave loads, with enough bytes in flight":
//   * W is packed once (mamba_linear_pack) into v_mfma_f32_32x32x16_bf16
//     B-operand order, 32-column tiles contiguous along K;
//   * the activation arrives already in A-operand order (written that way by
//     the producing kernel), so it too is read as contiguous 1 KB blocks (from
//     L2: it is small and shared by every workgroup);
//   * one workgroup owns one 32-column tile over a 1/S slice of K (grid.y =
//     S); its NW waves split that slice again, each software-pipelines its
//     loads two stages deep (stages of U k-steps, U chosen per launch from
//     the walk length, a last partial stage reading zero past the walk), and
//     the wave accumulators are reduced through LDS.  Small slices on many
//     workgroups (~1300) is what streams a weight at full HBM rate (a
//     workgroup's ramp-up and tail are then short); a product with few
//     column tiles may also split each tile into column parts (LinParams::CS);
//   * epilogues: plain store (+bias) when S = 1, else one f32 partial plane
//     per k-slice, summed in a fixed order by the consumer (deterministic, no
//     atomics).
#include <algorithm>

#include "lin.h"

namespace mamba {

typedef float lin_f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 lin_bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ lin_f32x16_t lin_mfma(lin_bf16x8_t a, lin_bf16x8_t b, lin_f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Tuning constants (compile-time; defaults measured on MI355X).
#ifndef MAMBA_LIN_NW
#define MAMBA_LIN_NW 4          // waves per workgroup for up to two 32-row tiles
#endif
#ifndef MAMBA_LIN_NW_BIGM
#define MAMBA_LIN_NW_BIGM 8     // waves per workgroup for four or eight 32-row tiles
#endif
#ifndef MAMBA_LIN_U1
#define MAMBA_LIN_U1 0          // k-steps per pipeline stage for one 32-row tile (0: lin_depth; 3..8)
#endif
#ifndef MAMBA_LIN_UMAX
#define MAMBA_LIN_UMAX 5        // deepest stage lin_depth picks for one 32-row tile (5, 6 or 8)
#endif
#ifndef MAMBA_LIN_U2
#define MAMBA_LIN_U2 0          // k-steps per pipeline stage for two 32-row tiles (0: lin_depth; 2..4)
#endif
#ifndef MAMBA_LIN_UMAX2
#define MAMBA_LIN_UMAX2 3       // deepest stage lin_depth picks for two 32-row tiles (3 or 4)
#endif
#ifndef MAMBA_LIN_NT
#define MAMBA_LIN_NT 0          // 1: weight loads carry the non-temporal hint (read once)
#endif
#ifndef MAMBA_LIN_ROTATE
#define MAMBA_LIN_ROTATE 0      // 1: each workgroup starts its k walk at a different stage
#endif

// One pipeline stage: U k-steps of weight and activation blocks.
template <int MT, int U>
struct LinStage {
    lin_bf16x8_t w[U];
    lin_bf16x8_t a[U][MT];
};
// k-steps per stage for four or eight 32-row tiles (their operands fill the registers)
template <int MT>
constexpr int lin_depth_fixed() { return MT == 4 ? 2 : 1; }

// Operand blocks through buffer resources (scalar base, 32-bit byte offsets):
// a load's address costs no 64-bit VGPR pair, which keeps the wave within the
// register budget of four waves per SIMD.
__device__ __forceinline__ lin_bf16x8_t lin_ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(lin_bf16x8_t, buf_ld16(r, off));
}

// Byte offset of activation block (s, i) for this lane: packed blocks are
// 1 KB runs; a row-major activation is read in place (lane -> row 32 i + r,
// k 16 s + 8 half .. + 7), rows past M beyond the resource's extent read zero.
template <int MT, bool RM>
struct LinAct {
    uint32_t lane_off, row_tile;  // RM: lane's (row r, k 8 half) offset; 32 rows of x
    __device__ __forceinline__ LinAct(int lane, int64_t x_ld) {
        if (RM) {
            lane_off = (uint32_t)(((int64_t)(lane & 31) * x_ld + 8 * (lane >> 5)) * 2);
            row_tile = (uint32_t)(32 * x_ld * 2);
        } else {
            lane_off = (uint32_t)lane * 16u;
            row_tile = 0;
        }
    }
    __device__ __forceinline__ uint32_t off(int s, int i) const {
        return RM ? lane_off + (uint32_t)i * row_tile + (uint32_t)s * 32u
                  : ((uint32_t)s * MT + i) * 1024u + lane_off;
    }
};

// Column parts per 32-column tile: 2 or 4 as asked, anything else one (a
// part count that does not divide the tile would leave columns unwritten).
__host__ __device__ __forceinline__ int lin_parts(const LinParams& p) { return p.CS == 2 || p.CS == 4 ? p.CS : 1; }

// A byte offset past every operand's extent: the load reads zero.
constexpr uint32_t kLinOut = 0x80000000u;

// One stage: k-steps s .. s + U - 1; those at or past s1 (the wave's end, in a
// last partial stage) read zero weights and activations, so they add nothing
// and every k-step of the wave is software-pipelined whatever U divides.
// `lo` is the lane's byte offset inside a weight block, or kLinOut for a lane
// whose column belongs to another column part (it then reads zero weights).
template <int MT, int U, bool RM>
__device__ __forceinline__ void lin_load(LinStage<MT, U>& st, __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t ra,
                                         uint32_t lo, const LinAct<MT, RM>& ao, int s, int s1) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool ok = s + u < s1;
        st.w[u] = lin_ld(rw, ok ? (uint32_t)(s + u) * 1024u + lo : kLinOut);
#pragma unroll
        for (int i = 0; i < MT; ++i) st.a[u][i] = lin_ld(ra, ok ? ao.off(s + u, i) : kLinOut);
    }
}

template <int MT, int U>
__device__ __forceinline__ void lin_compute(const LinStage<MT, U>& st, lin_f32x16_t (&acc)[MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i] = lin_mfma(st.a[u][i], st.w[u], acc[i]);
}

// grid: (ceil(N / 32), S) workgroups of NW waves.  RM: the activation is
// p.X (row-major bf16) instead of the packed p.A.  U: k-steps per stage.
template <int MT, int NW, int EPI, bool RM, int U>
__global__ __launch_bounds__(64 * NW) void lin_stream(LinParams p) {
    constexpr int RT = (MT < 2 || NW >= 16) ? 1 : 2;  // 32-row tiles reduced per LDS round
    __shared__ float s_red[NW][RT][16][64];
    const int cs = lin_parts(p);
    const int j = blockIdx.x / cs, z = blockIdx.y;
    const int cw = 32 / cs, c0 = (blockIdx.x % cs) * cw;  // this workgroup's columns 32 j + c0 ..
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int KS = p.K >> 4;
    const int z0 = (KS * z) / p.S, z1 = (KS * (z + 1)) / p.S;
    const int s0 = z0 + ((z1 - z0) * wave) / NW, s1 = z0 + ((z1 - z0) * (wave + 1)) / NW;

    // this tile's column of weight blocks, and the activation blocks
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(p.W + (int64_t)j * KS * 64, (uint32_t)KS * 1024u);
    const __amdgpu_buffer_rsrc_t ra = RM ? buf_rsrc(p.X, (uint32_t)((int64_t)p.M * p.x_ld * 2))
                                         : buf_rsrc(p.A, (uint32_t)KS * MT * 1024u);
    const LinAct<MT, RM> ao(lane, p.x_ld);
    const int lcol = lane & 31;
    uint32_t lo = (uint32_t)lane * 16u;
    lo = (lcol >= c0 && lcol < c0 + cw) ? lo : kLinOut;
    asm volatile("" : "+v"(lo));  // one select, not a branch around every load
    lin_f32x16_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;

    const int nstage = (s1 - s0 + U - 1) / U;  // the last stage may be partial
    if (nstage > 0) {
        // stage st covers k-steps s0 + U * ((st + rot) % nstage) .. + U - 1: with
        // rot varying over workgroups, concurrent waves read different blocks of
        // the (shared, L2-resident) activation instead of the same one
        const int rot = MAMBA_LIN_ROTATE ? (int)(blockIdx.x % (unsigned)nstage) : 0;
        auto kstep = [&](int st) { int q = st + rot; q -= q >= nstage ? nstage : 0; return s0 + U * q; };
        LinStage<MT, U> sa, sb;
        lin_load<MT, U, RM>(sa, rw, ra, lo, ao, kstep(0), s1);
        for (int st = 0; st < nstage; st += 2) {
            const bool more1 = st + 1 < nstage;
            if (more1) lin_load<MT, U, RM>(sb, rw, ra, lo, ao, kstep(st + 1), s1);
            lin_compute<MT, U>(sa, acc);
            if (more1) {
                if (st + 2 < nstage) lin_load<MT, U, RM>(sa, rw, ra, lo, ao, kstep(st + 2), s1);
                lin_compute<MT, U>(sb, acc);
            }
        }
    }

    // cross-wave reduction through LDS, RT 32-row tiles at a time
#pragma unroll
    for (int ig = 0; ig < MT; ig += RT) {
#pragma unroll
        for (int t2 = 0; t2 < RT; ++t2)
            if (ig + t2 < MT)
#pragma unroll
                for (int v = 0; v < 16; ++v) s_red[wave][t2][v][lane] = acc[ig + t2 < MT ? ig + t2 : 0][v];
        __syncthreads();
        for (int e = threadIdx.x; e < RT * 1024; e += 64 * NW) {
            const int t2 = e >> 10, v = (e >> 6) & 15, ln = e & 63;
            if (ig + t2 >= MT) break;
            const int m = 32 * (ig + t2) + 8 * (v >> 2) + 4 * (ln >> 5) + (v & 3);
            const int n = 32 * j + (ln & 31);
            if (m >= p.M || n >= p.N || (ln & 31) < c0 || (ln & 31) >= c0 + cw) continue;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) sum += s_red[w][t2][v][ln];
            if (EPI == LIN_STORE) {
                if (p.bias) sum += p.bias[n];
                if (p.out_bf16)
                    static_cast<bf16_t*>(p.out)[(int64_t)m * p.out_ld + n] = f32_to_bf16(sum);
                else
                    static_cast<float*>(p.out)[(int64_t)m * p.out_ld + n] = sum;
            } else {
                p.part[((int64_t)z * p.M + m) * p.N + n] = sum;
            }
        }
        __syncthreads();
    }
}

#ifndef MAMBA_LIN_GEMV
#define MAMBA_LIN_GEMV 1        // 1: products of one row take lin_gemv
#endif

// The product for one row (MM = 1; the code takes MM rows, M <= MM, but two
// rows measured slower than the MFMA kernel: 64-layer decode steps at batch 2
// 2.16 -> 2.19 ms for Mamba-2, 1.32 -> 1.40 ms for Mamba-3, against batch 1
// 2.08 -> 1.89 ms and 1.32 -> 1.28 ms): the same weight stream,
// plans and epilogues as lin_stream, but no MFMA.  A lane holds 8 k of one
// column of each weight block; the row's 8 matching activation values are one
// 16-byte load that every lane of the wave half shares (two addresses per wave
// and row, where the MFMA operand would be a 1 KB block whose other 31 rows
// are zero), and the products accumulate in f32 on the VALU by packed bf16
// dots (v_dot2c_f32_bf16: two products per instruction).  The two wave halves
// (k 0..7 and 8..15 of each block) are summed at the end.
template <int NW, int EPI, bool RM, int U, int MM>
__global__ __launch_bounds__(64 * NW) void lin_gemv(LinParams p) {
    __shared__ float s_red[NW][MM][32];
    const int cs = lin_parts(p);
    const int j = blockIdx.x / cs, z = blockIdx.y;
    const int cw = 32 / cs, c0 = (blockIdx.x % cs) * cw;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
    const int KS = p.K >> 4;
    const int z0 = (KS * z) / p.S, z1 = (KS * (z + 1)) / p.S;
    const int s0 = z0 + ((z1 - z0) * wave) / NW, s1 = z0 + ((z1 - z0) * (wave + 1)) / NW;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(p.W + (int64_t)j * KS * 64, (uint32_t)KS * 1024u);
    const __amdgpu_buffer_rsrc_t ra = RM ? buf_rsrc(p.X, (uint32_t)((int64_t)p.M * p.x_ld * 2))
                                         : buf_rsrc(p.A, (uint32_t)KS * 1024u);
    const int lcol = lane & 31;
    uint32_t lo = (uint32_t)lane * 16u;
    lo = (lcol >= c0 && lcol < c0 + cw) ? lo : kLinOut;
    asm volatile("" : "+v"(lo));
    // byte offset of row m's k = 16 s + 8 h .. + 7 (the packed operand of one row tile: lane m + 32 h)
    auto aoff = [&](int m, int s) -> uint32_t {
        return RM ? (uint32_t)(((int64_t)m * p.x_ld + 16 * s + 8 * h) * 2) : (uint32_t)((s * 64 + m + 32 * h) * 16);
    };
    struct Stage { uint4 w[U]; uint4 a[U][MM]; };
    auto load = [&](Stage& st, int s) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool ok = s + u < s1;
            st.w[u] = buf_ld16(rw, ok ? (uint32_t)(s + u) * 1024u + lo : kLinOut);
#pragma unroll
            for (int m = 0; m < MM; ++m) st.a[u][m] = buf_ld16(ra, ok && m < p.M ? aoff(m, s + u) : kLinOut);
        }
    };
    // four partial sums per row (k pairs e = 0..3 of each block), so that the
    // packed bf16 dots (two products into f32 per instruction) form four
    // independent chains
    float acc4[MM][4];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc4[m][e] = 0.f;
    auto compute = [&](const Stage& st) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t wv[4] = {st.w[u].x, st.w[u].y, st.w[u].z, st.w[u].w};
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const uint32_t xv[4] = {st.a[u][m].x, st.a[u][m].y, st.a[u][m].z, st.a[u][m].w};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc4[m][e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(lin_bf16x2_t, wv[e]),
                                                                 __builtin_bit_cast(lin_bf16x2_t, xv[e]), acc4[m][e], false);
            }
        }
    };
    const int nstage = (s1 - s0 + U - 1) / U;
    if (nstage > 0) {
        Stage sa, sb;
        load(sa, s0);
        for (int st = 0; st < nstage; st += 2) {
            const bool more1 = st + 1 < nstage;
            if (more1) load(sb, s0 + U * (st + 1));
            compute(sa);
            if (more1) {
                if (st + 2 < nstage) load(sa, s0 + U * (st + 2));
                compute(sb);
            }
        }
    }
    // the partial sums, the two halves of each column, then the waves
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        acc[m] = (acc4[m][0] + acc4[m][1]) + (acc4[m][2] + acc4[m][3]);
        acc[m] += __shfl_xor(acc[m], 32, 64);
    }
    if (lane < 32)
#pragma unroll
        for (int m = 0; m < MM; ++m) s_red[wave][m][lane] = acc[m];
    __syncthreads();
    if ((int)threadIdx.x < MM * 32) {
        const int m = threadIdx.x >> 5, c = threadIdx.x & 31, n = 32 * j + c;
        if (m < p.M && n < p.N && c >= c0 && c < c0 + cw) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) sum += s_red[w][m][c];
            if (EPI == LIN_STORE) {
                if (p.bias) sum += p.bias[n];
                if (p.out_bf16)
                    static_cast<bf16_t*>(p.out)[(int64_t)m * p.out_ld + n] = f32_to_bf16(sum);
                else
                    static_cast<float*>(p.out)[(int64_t)m * p.out_ld + n] = sum;
            } else {
                p.part[((int64_t)z * p.M + m) * p.N + n] = sum;
            }
        }
    }
}

template <int NW, bool RM, int U, int MM>
static void lin_launch_gemv(const LinParams& p, int epi, hipStream_t stream) {
    const dim3 grid(((p.N + 31) / 32) * lin_parts(p), p.S);
    if (epi == LIN_STORE) hipLaunchKernelGGL((lin_gemv<NW, LIN_STORE, RM, U, MM>), grid, dim3(64 * NW), 0, stream, p);
    else hipLaunchKernelGGL((lin_gemv<NW, LIN_PARTIAL, RM, U, MM>), grid, dim3(64 * NW), 0, stream, p);
}

template <int MT, int NW, bool RM, int U>
static void lin_launch_u(const LinParams& p, int epi, hipStream_t stream) {
    const dim3 grid(((p.N + 31) / 32) * lin_parts(p), p.S);
    if (epi == LIN_STORE) hipLaunchKernelGGL((lin_stream<MT, NW, LIN_STORE, RM, U>), grid, dim3(64 * NW), 0, stream, p);
    else hipLaunchKernelGGL((lin_stream<MT, NW, LIN_PARTIAL, RM, U>), grid, dim3(64 * NW), 0, stream, p);
}

// Stage depth from kw, the most k-steps a wave walks: at least two stages (one
// would leave nothing to overlap), as few masked k-steps in the last stage as
// possible, and of those the deepest stage in [umin, umax] (the most weight
// bytes in flight per wave).  At a fixed depth of 3 a wave's walk of 8
// k-steps ran its last two outside the pipeline; chosen this way (depth 4 for
// walks of 8, 5 for walks of 10 and 20) the 64-layer decode steps went 3.36 ->
// 3.07 ms (Mamba-3, batch 64), 1.38 -> 1.30 ms (batch 1) and 5.87 -> 5.78 ms
// (Mamba-2, batch 64), 3.03 -> 2.97 ms (batch 16).
static int lin_depth(int kw, int umax, int umin) {
    int best = umin, waste = 1 << 30;
    for (int u = umax; u >= umin; --u) {
        const int ns = (kw + u - 1) / u;
        if (ns < 2) continue;
        if (ns * u - kw < waste) {
            waste = ns * u - kw;
            best = u;
        }
    }
    return best;
}

template <int MT, int NW, bool RM>
static void lin_launch_nw(const LinParams& p, int epi, hipStream_t stream) {
    const int ks = p.K >> 4, kz = (ks + p.S - 1) / p.S, kw = (kz + NW - 1) / NW;
    if constexpr (MT == 1) {
        if (MAMBA_LIN_GEMV && p.M == 1) {
            const int ug = lin_depth(kw, 5, 3);
            if (ug == 5) lin_launch_gemv<NW, RM, 5, 1>(p, epi, stream);
            else if (ug == 4) lin_launch_gemv<NW, RM, 4, 1>(p, epi, stream);
            else lin_launch_gemv<NW, RM, 3, 1>(p, epi, stream);
            return;
        }
        // 16 waves (at most 128 registers each) hold stages of up to 6 k-steps
        const int u = MAMBA_LIN_U1 ? MAMBA_LIN_U1 : lin_depth(kw, NW >= 16 ? std::min(MAMBA_LIN_UMAX, 6) : MAMBA_LIN_UMAX, 3);
        switch (u) {
#if MAMBA_LIN_UMAX >= 8
            case 8: if constexpr (NW < 16) { lin_launch_u<1, NW, RM, 8>(p, epi, stream); return; }
            [[fallthrough]];
            case 7: if constexpr (NW < 16) { lin_launch_u<1, NW, RM, 7>(p, epi, stream); return; }
            [[fallthrough]];
#endif
#if MAMBA_LIN_UMAX >= 6
            case 6: lin_launch_u<1, NW, RM, 6>(p, epi, stream); return;
#endif
            case 5: lin_launch_u<1, NW, RM, 5>(p, epi, stream); return;
            case 4: lin_launch_u<1, NW, RM, 4>(p, epi, stream); return;
            default: lin_launch_u<1, NW, RM, 3>(p, epi, stream); return;
        }
    } else if constexpr (MT == 2) {
        const int u = MAMBA_LIN_U2 ? MAMBA_LIN_U2 : lin_depth(kw, NW >= 16 ? 3 : MAMBA_LIN_UMAX2, 2);
        switch (u) {
#if MAMBA_LIN_UMAX2 >= 4
            case 4: if constexpr (NW < 16) { lin_launch_u<2, NW, RM, 4>(p, epi, stream); return; }
            [[fallthrough]];
#endif
            case 3: lin_launch_u<2, NW, RM, 3>(p, epi, stream); return;
            default: lin_launch_u<2, NW, RM, 2>(p, epi, stream); return;
        }
    } else {
        lin_launch_u<MT, NW, RM, lin_depth_fixed<MT>()>(p, epi, stream);
    }
}

template <int MT>
static void lin_launch_mt(const LinParams& p, int epi, hipStream_t stream) {
    constexpr int NWD = MT <= 2 ? MAMBA_LIN_NW : MAMBA_LIN_NW_BIGM;
    const int nw = p.NW ? p.NW : NWD;
    const bool rm = p.X != nullptr;
    if constexpr (MT <= 2) {
        // 16 waves (1024 threads, at most 128 registers each) only for up to
        // two 32-row tiles, whose accumulators and operand stages fit
        if (nw == 16) {
            if (rm) lin_launch_nw<MT, 16, true>(p, epi, stream);
            else lin_launch_nw<MT, 16, false>(p, epi, stream);
            return;
        }
    }
    if (nw >= 8) {
        if (rm) lin_launch_nw<MT, 8, true>(p, epi, stream);
        else lin_launch_nw<MT, 8, false>(p, epi, stream);
    } else {
        if (rm) lin_launch_nw<MT, 4, true>(p, epi, stream);
        else lin_launch_nw<MT, 4, false>(p, epi, stream);
    }
}

void lin_launch(const LinParams& p, int epi, hipStream_t stream) {
    switch (p.MT) {
        case 1: lin_launch_mt<1>(p, epi, stream); break;
        case 2: lin_launch_mt<2>(p, epi, stream); break;
        case 4: lin_launch_mt<4>(p, epi, stream); break;
        default: lin_launch_mt<8>(p, epi, stream); break;
    }
}

// ---------------------------------------------------------------------------
// Weight packing: W [K, N] row-major (Burn Linear layout [d_in, d_out]), f32 or
// bf16, into the packed bf16 B-operand format; columns past N are zero.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void lin_pack_kernel(const void* W, int K, int N, int64_t ldw, bool w_bf16,
                                                       lin_bf16x8_t* out) {
    const int64_t KS = K / 16;
    const int64_t nlanes = (int64_t)((N + 31) / 32) * KS * 64;
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < nlanes; g += (int64_t)gridDim.x * 256) {
        const int lane = (int)(g & 63);
        const int64_t blk = g >> 6;
        const int j = (int)(blk / KS), s = (int)(blk % KS);
        const int n = 32 * j + (lane & 31);
        const int k0 = 16 * s + 8 * (lane >> 5);
        lin_bf16x8_t v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float f = 0.f;
            if (n < N) {
                const int64_t idx = (int64_t)(k0 + e) * ldw + n;
                f = w_bf16 ? bf16_to_f32(static_cast<const bf16_t*>(W)[idx]) : static_cast<const float*>(W)[idx];
            }
            v[e] = (__bf16)f;
        }
        out[g] = v;
    }
}

}  // namespace mamba

using namespace mamba;

extern "C" size_t mamba_linear_packed_size(int32_t d_in, int32_t d_out) {
    if (d_in <= 0 || d_out <= 0 || d_in % 16 != 0) return 0;
    return lin_weight_elems(d_in, d_out) * 2;
}

extern "C" int mamba_linear_pack(const void* weight, int32_t d_in, int32_t d_out, int64_t ld, int32_t dtype,
                                 void* packed, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(weight && packed, "weight and packed are required");
    MAMBA_CHECK_ARG(d_in > 0 && d_out > 0, "d_in and d_out must be >= 1");
    MAMBA_CHECK_ARG(d_in % 16 == 0, "d_in must be a multiple of 16");
    MAMBA_CHECK_ARG(ld >= d_out, "ld must be >= d_out");
    MAMBA_CHECK_ARG(dtype == MAMBA_F32 || dtype == MAMBA_BF16, "bad dtype");
    MAMBA_CHECK_ARG(((uintptr_t)packed & 15u) == 0, "packed must be 16-byte aligned");
    const int64_t nlanes = (int64_t)((d_out + 31) / 32) * (d_in / 16) * 64;
    const int grid = (int)std::min<int64_t>((nlanes + 255) / 256, 8192);
    hipLaunchKernelGGL(lin_pack_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, weight, d_in, d_out, ld,
                       dtype == MAMBA_BF16, static_cast<lin_bf16x8_t*>(packed));
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

// ---------------------------------------------------------------------------
// General entry: y = x W (+bias) with x row-major; x is packed into the
// workspace first (one 16-byte run of 8 consecutive k per thread).
// ---------------------------------------------------------------------------
namespace mamba {

__global__ __launch_bounds__(256) void lin_act_pack_kernel(const void* x, int M, int K, int64_t ldx, bool x_bf16,
                                                           bf16_t* a_out, int mt) {
    const int groups = K / 8;
    const int64_t total = (int64_t)M * groups;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
        const int m = (int)(idx / groups), g = (int)(idx % groups);
        uint32_t u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t i0 = (int64_t)m * ldx + 8 * g + 2 * e;
            float f0, f1;
            if (x_bf16) {
                f0 = bf16_to_f32(static_cast<const bf16_t*>(x)[i0]);
                f1 = bf16_to_f32(static_cast<const bf16_t*>(x)[i0 + 1]);
            } else {
                f0 = static_cast<const float*>(x)[i0];
                f1 = static_cast<const float*>(x)[i0 + 1];
            }
            u[e] = (uint32_t)f32_to_bf16(f0) | ((uint32_t)f32_to_bf16(f1) << 16);
        }
        *reinterpret_cast<uint4*>(a_out + lin_act_offset(m, 8 * g, mt)) = make_uint4(u[0], u[1], u[2], u[3]);
    }
}

}  // namespace mamba

namespace mamba {

// y[m, n] = sum_z part[z][m][n] (+ bias[n]), planes summed in order.
__global__ __launch_bounds__(256) void lin_reduce_kernel(const float* part, int S, int M, int N, const float* bias,
                                                         void* y, int64_t y_ld, bool y_bf16) {
    const int64_t total = (int64_t)M * N;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
        const int m = (int)(idx / N), n = (int)(idx % N);
        float v = bias ? bias[n] : 0.f;
        for (int z = 0; z < S; ++z) v += part[(int64_t)z * total + idx];
        if (y_bf16)
            static_cast<bf16_t*>(y)[(int64_t)m * y_ld + n] = f32_to_bf16(v);
        else
            static_cast<float*>(y)[(int64_t)m * y_ld + n] = v;
    }
}

// The entry's plan for one product.  A bf16 row-major x with 16-byte aligned
// rows is read in place (no packing pass).  With one 32-row tile (rows <= 32),
// weights up to LINFWD_ONE_SPLIT bytes are streamed with one k-split, so the
// product writes y directly (no partial planes, no summing pass), with enough
// waves per workgroup for LINFWD_MIN_WAVES streaming waves.  Measured on the
// 64-layer Mamba-3 decode step (in_proj 10.8 MB, out_proj 4.2 MB): at batch 1
// this takes the step from 1.59 to 1.45 ms, while at batch 64 (two row tiles)
// the one-split product is slower than the k-split one plus its summing pass
// (4.09 against 3.80 ms), so larger batches keep the k-split plan.
#ifndef MAMBA_LINFWD_RM
#define MAMBA_LINFWD_RM 1
#endif
#ifndef MAMBA_LINFWD_ONE_SPLIT
#define MAMBA_LINFWD_ONE_SPLIT (16ll << 20)
#endif
#ifndef MAMBA_LINFWD_ONE_SPLIT_MT
#define MAMBA_LINFWD_ONE_SPLIT_MT 1
#endif
#ifndef MAMBA_LINFWD_MIN_WAVES
#define MAMBA_LINFWD_MIN_WAVES 1024
#endif
#ifndef MAMBA_LINFWD_MAX_CS
#define MAMBA_LINFWD_MAX_CS 4
#endif
struct LinPlan {
    bool rm;  // x read in place
    int S, NW, CS;
};

static LinPlan linear_plan(const mamba_linear_args* a) {
    LinPlan pl;
    pl.rm = MAMBA_LINFWD_RM && a->x_dtype == MAMBA_BF16 && a->x_ld % 8 == 0 && ((uintptr_t)a->x & 15u) == 0 &&
            (int64_t)a->rows * a->x_ld * 2 < (1ll << 31);
    const int mt = lin_mt(a->rows), tiles = (a->d_out + 31) / 32, ks = a->d_in / 16;
    if (mt <= MAMBA_LINFWD_ONE_SPLIT_MT && (int64_t)a->d_in * tiles * 32 * 2 <= MAMBA_LINFWD_ONE_SPLIT) {
        pl.S = 1;
        const int nw_max = mt <= 2 ? 16 : 8;
        int nw = 4;
        while (nw < nw_max && tiles * nw < MAMBA_LINFWD_MIN_WAVES && ks / (2 * nw) >= 3) nw *= 2;
        pl.NW = nw;
        // few column tiles even at the widest workgroups (out_proj, d_out =
        // d_model): column parts, still one pass and no partial planes
        int cs = 1;
        while (cs < MAMBA_LINFWD_MAX_CS && tiles * nw * cs < MAMBA_LINFWD_MIN_WAVES) cs *= 2;
        pl.CS = cs;
    } else {
        pl.S = lin_splits(a->rows, a->d_in, a->d_out);
        pl.NW = 0;
        pl.CS = 1;
    }
    return pl;
}

static size_t linear_ws(const mamba_linear_args* a, size_t* part_off) {
    const LinPlan pl = linear_plan(a);
    const size_t act = pl.rm ? 0 : align_up(lin_act_elems(a->rows, a->d_in) * 2, 256);
    *part_off = act;
    return act + (pl.S > 1 ? align_up(lin_part_elems(a->rows, a->d_out, pl.S) * 4, 256) : 0);
}

}  // namespace mamba

extern "C" size_t mamba_linear_workspace_size(const mamba_linear_args* a) {
    if (a == nullptr || a->rows <= 0 || a->d_in <= 0 || a->d_out <= 0) return 0;
    size_t off;
    return linear_ws(a, &off);
}

extern "C" int mamba_linear_fwd(const mamba_linear_args* a, void* ws, size_t ws_bytes, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->rows >= 1 && a->rows <= 256, "rows must be in [1, 256]");
    MAMBA_CHECK_ARG(a->d_in > 0 && a->d_in % 16 == 0 && a->d_out > 0, "d_in must be a positive multiple of 16");
    MAMBA_CHECK_ARG(a->x && a->packed_w && a->y, "x, packed_w and y are required");
    MAMBA_CHECK_ARG(a->x_dtype == MAMBA_F32 || a->x_dtype == MAMBA_BF16, "bad x_dtype");
    MAMBA_CHECK_ARG(a->y_dtype == MAMBA_F32 || a->y_dtype == MAMBA_BF16, "bad y_dtype");
    MAMBA_CHECK_ARG(a->x_ld >= a->d_in && a->y_ld >= a->d_out, "leading dimensions too small");
    MAMBA_CHECK_ARG(((uintptr_t)a->packed_w & 15u) == 0, "packed_w must be 16-byte aligned");
    size_t part_off;
    const size_t need = linear_ws(a, &part_off);
    if ((need > 0 && ws == nullptr) || ws_bytes < need || ((uintptr_t)ws & 15u) != 0) {
        set_error("mamba_linear_fwd: a 16-byte aligned workspace of " + std::to_string(need) + " bytes is required");
        return MAMBA_ERR_WORKSPACE;
    }
    const int mt = lin_mt(a->rows);
    hipStream_t s = (hipStream_t)stream;
    const LinPlan pl = linear_plan(a);
    LinParams p = {};
    p.M = a->rows; p.N = a->d_out; p.K = a->d_in; p.MT = mt; p.S = pl.S; p.NW = pl.NW; p.CS = pl.CS;
    p.W = static_cast<const lin_bf16x8_t*>(a->packed_w);
    if (pl.rm) {
        p.X = static_cast<const bf16_t*>(a->x);
        p.x_ld = a->x_ld;
    } else {
        const int64_t total = (int64_t)a->rows * (a->d_in / 8);
        hipLaunchKernelGGL(lin_act_pack_kernel, dim3((int)std::min<int64_t>((total + 255) / 256, 4096)), dim3(256), 0,
                           s, a->x, a->rows, a->d_in, a->x_ld, a->x_dtype == MAMBA_BF16, static_cast<bf16_t*>(ws), mt);
        MAMBA_CHECK_LAUNCH();
        p.A = static_cast<const lin_bf16x8_t*>(ws);
    }
    if (p.S == 1) {
        p.bias = a->bias;
        p.out = a->y; p.out_ld = a->y_ld; p.out_bf16 = a->y_dtype == MAMBA_BF16;
        lin_launch(p, LIN_STORE, s);
        MAMBA_CHECK_LAUNCH();
        return MAMBA_OK;
    }
    p.part = reinterpret_cast<float*>(static_cast<char*>(ws) + part_off);
    lin_launch(p, LIN_PARTIAL, s);
    MAMBA_CHECK_LAUNCH();
    const int64_t nout = (int64_t)a->rows * a->d_out;
    hipLaunchKernelGGL(lin_reduce_kernel, dim3((int)std::min<int64_t>((nout + 255) / 256, 4096)), dim3(256), 0, s,
                       p.part, p.S, a->rows, a->d_out, a->bias, a->y, a->y_ld, a->y_dtype == MAMBA_BF16);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}
