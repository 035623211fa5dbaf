// Mamba-2 chunked SSD forward, gfx950 MFMA path (bf16 in/out, f32 state).
//
// Reference: src/mamba2/ssd/serial.rs:34-506 (K1 cumsum, K2 C.B^T, K3 chunk
// state, K4 state passing, K5 chunk scan) and the trait default body
// src/mamba2/ssd/serial_recalculated/serial_recalculated.rs:98-155.
//
// Two launches per call:
//   1. ssd2_prep_pack (per batch, chunk, group): the group-shared causal
//      C_c.B_c^T tiles (K2, computed once per group instead of once per head,
//      f32 accumulation rounded to bf16), C_c and B_c in bf16, written as one
//      packed run of 1 KB MFMA operand fragments per (batch, chunk, group).
//   2. ssd2_scan_wu: one wave per (batch, head, 32-wide headdim half) walks
//      the chunks in order, with the running state in its MFMA accumulators
//      for the whole sequence (K4 needs no HBM round trip).  The HPW waves of
//      a workgroup are HPW heads of one group: the only thing they share is
//      the group's fragments, which the workgroup stages once per chunk into
//      LDS with direct-to-LDS loads (double-buffered, one barrier per chunk).
//      Per chunk a wave computes K1 in its lanes, then
//        y = exp(cs_i) C_i . h_in + sum_{j<=i} (C_i.B_j) dt_j exp(cs_i-cs_j) x_j + D x_i
//        h_out = exp(cs_end) h_in + sum_j (B_j dt_j exp(cs_end - cs_j)) (x) x_j
//      with every contraction on v_mfma_f32_32x32x16_bf16.  x is read from
//      HBM once, y is written once.
//
// MFMA 32x32x16 operand/result layout (lane l, r = l % 32, half = l / 32):
//   A[m][k]: lane holds row m = r, k = 8*half .. 8*half+7
//   B[k][n]: lane holds col n = r, k = 8*half .. 8*half+7
//   D[m][n]: lane holds col n = r, rows 8*(v/4) + 4*half + (v%4), v = 0..15
// Any permutation of k that A and B share leaves the product unchanged; the
// row/col mappings and the D layout are what the indexing below relies on.

#include <cstdlib>

#include "ssd2.h"

namespace mamba {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxQ = 256;

#ifndef MAMBA_SSD2_L2_WARM
#define MAMBA_SSD2_L2_WARM 1  // touch the chunk after next's fragments ahead of use
#endif

__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 8 packed bf16 (one uint4) -> 8 floats
__device__ __forceinline__ void unpack8(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[2 * k] = __uint_as_float(w[k] << 16);
        f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}

__device__ __forceinline__ bf16x8_t pack8(const float* f) {
    bf16x8_t r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (__bf16)f[e];
    return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
    return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x16_t zero16() {
    f32x16_t z;
#pragma unroll
    for (int v = 0; v < 16; ++v) z[v] = 0.f;
    return z;
}

// Fragments per (batch, chunk, group), in the order the scan kernel stages them:
//   CB  it*(it+1) + ks         (C.B^T)[i = 32 it + lane%32][j = 16 ks + 8 (lane/32) + e],
//                              ks <= 2 it + 1 (the causal ones)
//   C   NCB + it*NK + kn       C[i = 32 it + lane%32][n = 16 kn + perm(lane/32, e)]
//   B   NCB + T*NK + nt*KS+ks  B[j = 16 ks + 8 (lane/32) + e][n = 32 nt + lane%32]
// each 64 lanes x 8 bf16 = 1 KB.  perm(half, e) = e < 4 ? 4 half + e : 8 + 4 half + e - 4
// is the k order in which a wave's state accumulator rows (D layout) sit in its
// lanes, so the state enters h . C^T as the A operand straight from registers.
template <int N, int Q>
struct FragLayout {
    static constexpr int T = Q / 32, NK = N / 16, KS = Q / 16, NTN = N / 32;
    static constexpr int NCB = T * (T + 1);
    static constexpr int C0 = NCB, B0 = NCB + T * NK;
    static constexpr int NF = B0 + NTN * KS;
};

// ------------------------------------------------ per-group operand prep --
// Per (batch, chunk, group) -- shared by every head of the group -- write the
// fragments above.  Positions past seqlen read as zero.  Only the causal
// (ks <= 2 it + 1) C.B^T fragments are written (K2, src/mamba2/ssd/serial.rs:170-185),
// and inside the diagonal 32x32 blocks the entries with j > i are stored as 0.
// One workgroup per (chunk, group, batch): the chunk's B and C rows are read
// once into LDS with 16-byte loads (rows padded by 16 bytes, so that the
// transposed reads of the B fragments and the row reads of the C.B^T
// operands spread over the banks), then every fragment is formed from LDS
// and written as one contiguous 1 KB run.
template <int N, int Q>
__global__ __launch_bounds__(256) void ssd2_prep_pack(Ssd2Params p, bf16_t* frag) {
    using FL = FragLayout<N, Q>;
    constexpr int T = FL::T, NK = FL::NK, KS = FL::KS, NTN = FL::NTN, NF = FL::NF;
    constexpr int NTILE = T * (T + 1) / 2;
    constexpr int RP = N + 8;                  // LDS row pitch (bf16)
    constexpr int PR = N / 8;                  // 16-byte pieces per row
    __shared__ __align__(16) bf16_t sB[Q][RP];
    __shared__ __align__(16) bf16_t sC[Q][RP];
    const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, r = lane & 31, half = lane >> 5;
    const int cg = blockIdx.x, c = cg / p.G, g = cg % p.G, b = blockIdx.y;
    const int64_t grp = ((int64_t)b * p.nch + c) * p.G + g;
    const bf16_t* Cg = (const bf16_t*)p.Cm + (int64_t)b * p.C_sb + (int64_t)g * p.C_sg;
    const bf16_t* Bg = (const bf16_t*)p.Bm + (int64_t)b * p.B_sb + (int64_t)g * p.B_sg;
    bf16_t* base = frag + grp * NF * 512;
    // ---- the chunk's B and C rows into LDS (rows past seqlen as zero)
#pragma unroll
    for (int k = 0; k < (2 * Q * PR + 255) / 256; ++k) {
        const int pi = tid + 256 * k;
        if (pi < 2 * Q * PR) {
            const int arr = pi / (Q * PR), row = (pi / PR) % Q, col = (pi % PR) * 8;
            const int t = c * Q + row;
            const bf16_t* src = (arr ? Cg + (int64_t)t * p.C_sl : Bg + (int64_t)t * p.B_sl) + col;
            const uint4 v = t < p.L ? *(const uint4*)src : make_uint4(0u, 0u, 0u, 0u);
            *(uint4*)(arr ? &sC[row][col] : &sB[row][col]) = v;
        }
    }
    __syncthreads();
    // ---- (C.B^T)^T tiles: D[j][i] = sum_n B[j][n] C[i][n]; the lane then holds
    // column i = 32 it + r at rows j = 32 jt + 8 q + 4 half + u (v = 4 q + u)
    for (int tile = wave; tile < NTILE; tile += 4) {
        int it = 0;
        while ((it + 1) * (it + 2) / 2 <= tile) ++it;
        const int jt = tile - it * (it + 1) / 2;
        f32x16_t acc = zero16();
#pragma unroll
        for (int kn = 0; kn < NK; ++kn) {
            const int n0 = kn * 16 + 8 * half;
            acc = mfma32x32x16(as_bf16x8(*(const uint4*)&sB[jt * 32 + r][n0]),
                               as_bf16x8(*(const uint4*)&sC[it * 32 + r][n0]), acc);
        }
        if (jt == it) {  // causal mask of the diagonal block: row j = 8 q + 4 half + u, column i = r
#pragma unroll
            for (int v = 0; v < 16; ++v)
                if (8 * (v >> 2) + 4 * half + (v & 3) > r) acc[v] = 0.f;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ks = 2 * jt + (q >> 1), lp = r + 32 * (q & 1);
            // fragment (it, ks), lane lp, elements 4 half .. 4 half + 3
            uint2 pk;
            pk.x = pack_bf16x2(acc[4 * q], acc[4 * q + 1]);
            pk.y = pack_bf16x2(acc[4 * q + 2], acc[4 * q + 3]);
            *(uint2*)(base + ((int64_t)(it * (it + 1) + ks) * 64 + lp) * 8 + 4 * half) = pk;
        }
    }
    // ---- C fragments (k order perm(half, .)) and B fragments (transposed)
    for (int f = wave; f < T * NK + NTN * KS; f += 4) {
        uint4 v;
        if (f < T * NK) {
            const int it = f / NK, kn = f % NK;
            const bf16_t* row = &sC[it * 32 + r][kn * 16 + 4 * half];
            const uint2 lo = *(const uint2*)row, hi = *(const uint2*)(row + 8);
            v = make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else {
            const int fb = f - T * NK, nt = fb / KS, ks = fb % KS;
            const int n = nt * 32 + r, j0 = ks * 16 + 8 * half;
            uint32_t raw[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) raw[e] = (uint32_t)sB[j0 + e][n];
            v = make_uint4(raw[0] | (raw[1] << 16), raw[2] | (raw[3] << 16), raw[4] | (raw[5] << 16),
                           raw[6] | (raw[7] << 16));
        }
        *(uint4*)(base + ((int64_t)(FL::C0 + f) * 64 + lane) * 8) = v;
    }
}

// ----------------------------------------------- K1 + K3 + K4 + K5 fused --
// One wave per (batch, head, 32-wide headdim half), HPW waves (HPW heads of
// one group) per workgroup; chunks in order.  N = dstate, Q = chunk length
// (32 or 64: a chunk's positions are the wave's lanes).
//
// The state is carried transposed, h^T[n, p] (n along MFMA rows, p along
// columns), in NTN accumulator tiles: the state GEMM is h^T += B^T . xg with
// the B fragments as the A operand and xg from LDS as the B operand, and the
// accumulator registers of h^T, converted to bf16 eight at a time, are the A
// operand of y^T = h . C^T (the C fragments carry the matching k order).  So
// nothing of the state leaves the registers between chunks.
//
// The chunk is cut into 32-position blocks k = 0 .. T-1 ending at e_k = 32k+31
// (cs_{e_-1} = 0 is the chunk start).  Every decay is carried by x and by a
// scalar recurrence, so that the group-shared fragments (C.B^T, C, B) enter
// the MFMAs exactly as the prep stored them, with no per-element work:
//   xg_j = x_j dt_j exp(cs_{e_k} - cs_j)          (j in block k; factor <= 1)
//   F_k  = exp(cs_{e_k} - cs_{e_{k-1}})           (block decay; <= 1)
//   S_k[i] = sum_{j in k} (C_i.B_j) xg_j           (raw C.B^T fragments)
// Output block `it` is then a Horner recurrence over the blocks before it,
//   acc = C_i.h_in;  acc = acc F_k + S_k  (k = 0 .. it)
//   y_i = exp(cs_i - cs_{e_it}) acc + D x_i
// and the chunk state is the same recurrence over all T blocks with the raw B
// fragments,  h <- h F_k + sum_{j in k} B_j (x) xg_j.
// The decays are applied lazily: the registers hold h-hat with h = phi h-hat
// for a wave-uniform phi (kept as log2), so that h <- h F_k is phi <- phi F_k
// and S_k enters as S_k / phi (1 / phi folded into xg, the Horner
// accumulators likewise in phi units, phi folded into the output factor).
// Only when phi would drop below 2^-64 is it applied to the registers (an
// "event": h-hat and the live accumulators times phi, phi = 1), which bounds
// xg / phi and h-hat by 2^64 times their true size.
// xg^T is kept in LDS as the MFMA operand, and the raw x rows (time-major)
// for the D x_i term.  The output's last factor exp(cs_i - cs_{e_it}) is >= 1
// and xg_j of the diagonal block can be as small as exp(cs_{e_it} -
// cs_{e_{it-1}}); when that block decay exceeds 2^-64 (a steep block) the
// tile is recomputed with the exact per-element weight dt_j exp(cs_i - cs_j)
// on the diagonal block, after scaling acc by exp(cs_i - cs_{e_{it-1}}) <= 1.
// Raw x is read back from global memory on that rare path only.
//
// Outputs are computed transposed, y^T[p, i] (i = time along MFMA columns),
// so every per-time factor is a per-lane scalar and the four consecutive
// headdim values a lane holds are stored as one 8-byte write.
//
// Per chunk c a wave: issues the direct-to-LDS loads of its share of chunk
// c + 1's fragments (into the other buffer); stores chunk c - 1's outputs;
// scans dt; stages xg and the raw x rows; issues its register prefetch of
// chunk c + 1's x rows and dt; computes its output tiles and its state; then
// waits for its loads and meets the others at the chunk's one barrier, after
// which chunk c + 1's fragments are complete and chunk c's buffer is free.
// The launch bound caps a wave at 256 registers (two waves per SIMD), which
// keeps the accumulators in VGPRs next to the VALU work that scales them.
template <int N, int Q, int HPW>
__global__ __launch_bounds__(64 * HPW, HPW >= 5 ? 1 : 8 / HPW) void ssd2_scan_wu(Ssd2Params p, const bf16_t* frag) {
    using FL = FragLayout<N, Q>;
    constexpr int T = FL::T, NK = FL::NK, KS = FL::KS, NTN = FL::NTN, NF = FL::NF;
    constexpr int XP = Q + 8;                 // s_xg row pitch (bf16)
    constexpr int XPT = Q / 32;               // x staging items per lane: (2 rows x 8 headdim) each
    constexpr int FPW = (NF + HPW - 1) / HPW; // fragments each wave stages per chunk
    constexpr float kSteep = 64.f;            // log2 of the largest block decay factored
    constexpr float kLazy = 64.f;             // log2 of the smallest pending state factor
    static_assert(Q == 32 || Q == 64, "a chunk's positions are the wave's lanes");
    // the group's fragments of two chunks, as two arrays: the reads of one and
    // the direct-to-LDS loads into the other are then provably disjoint, so no
    // wait for those loads is placed before the reads
    __shared__ __align__(16) bf16_t s_fragA[NF][512];
    __shared__ __align__(16) bf16_t s_fragB[NF][512];
    __shared__ __align__(16) bf16_t s_xg[HPW][32][XP];   // per wave: xg^T [p][j]
    __shared__ __align__(16) float s_cs[HPW][Q];         // per wave: cumsum (log2 units)
    __shared__ __align__(16) float s_dt[HPW][Q];         // per wave: dt
    // per wave: the chunk's raw x rows, time-major, overwritten in place by
    // its output rows (stored to global memory at the start of the next
    // chunk).  A row's 32 headdim values sit in MFMA-result order, headdim
    // p at 16 ((p / 4) % 2) + 4 (p / 8) + p % 4, so that the 16 values a
    // lane holds of a row are contiguous (two 16-byte accesses)
    __shared__ __align__(16) bf16_t s_io[HPW][T][32][40];

    const int wave = wave_id(), lane0 = threadIdx.x & 63;
    // XCD-aware work mapping: consecutive workgroups (same batch row, sharing
    // its group fragments through L2) land on the same XCD
    const int nhq = p.H / HPW;                // head sets per batch row
    const int nwg = p.nb * nhq * 2;
    int w = blockIdx.x;
    if ((nwg & 7) == 0) w = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    const int ph = w & 1, hq = (w >> 1) % nhq, b = (w >> 1) / nhq;
    const int hpg = p.H / p.G;
    const int g = (hq * HPW) / hpg;           // all HPW heads of the workgroup are in group g
    const int h = hq * HPW + wave;            // this wave's head
    const int p0 = ph * 32;
    const float A2 = p.A[h] * kLog2e;
    const float Dh = p.D ? p.D[h] : 0.f;

    // ---- the state h^T: tile nt, register v holds (n = 32 nt + 8 (v/4) + 4 half + v%4, p = p0 + r)
    f32x16_t hacc[NTN];
    {
        const int r = lane0 & 31, half = lane0 >> 5;
        const int64_t hrow = (((int64_t)b * p.H + h) * 64 + p0 + r) * N;
        const float* hin = p.h0 ? p.h0 + hrow : nullptr;
        const float* hid = p.init_hpr ? p.init_hpr + ((int64_t)h * 64 + p0 + r) * N : nullptr;
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = 32 * nt + 8 * q + 4 * half;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (hin) v = *(const float4*)(hin + n);
                if (hid) {
                    const float4 u = *(const float4*)(hid + n);
                    v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
                }
                hacc[nt][4 * q] = v.x; hacc[nt][4 * q + 1] = v.y;
                hacc[nt][4 * q + 2] = v.z; hacc[nt][4 * q + 3] = v.w;
            }
    }

    const bf16_t* xhead = (const bf16_t*)p.x + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh + p0;
    const float* dthead = p.dt + (int64_t)b * p.dt_sb + (int64_t)h * p.dt_sh;
    bf16_t* yhead = (bf16_t*)p.y + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh + p0;
    const uint32_t xrow = (uint32_t)p.x_sl * 2u;
    const int64_t grp_stride = (int64_t)p.G * NF * 512;       // bf16 elements per chunk step
    const bf16_t* gfrag = frag + ((int64_t)b * p.nch * p.G + g) * NF * 512;  // chunk 0 of (b, g)

    // direct-to-LDS loads of chunk cc's fragments f = wave + HPW k into `dst`
    auto stage = [&](int cc, bf16_t (&dst)[NF][512], int lane) __attribute__((always_inline)) {
        const u32x4_t rf = buf_words(gfrag + (int64_t)cc * grp_stride, (uint32_t)NF * 1024u);
#pragma unroll
        for (int k = 0; k < FPW; ++k) {
            const int f = wave + HPW * k;
            if (FPW * HPW == NF || f < NF)
                dma16(rf, (uint32_t)(uintptr_t)&dst[f][0], lane * 16u,
                      (uint32_t)__builtin_amdgcn_readfirstlane(f * 1024));
        }
    };
    // register prefetch of chunk cc's x rows (item m: rows 2 (lane/4 + 16 m) + {0, 1},
    // headdim vector lane % 4) and dt (lane = position); loads past the end read zero.
    // x is read once: its loads carry the non-temporal hint, which keeps the
    // group fragments (shared by every workgroup of the group) resident in L2
    uint4 xq[XPT][2];
    float dtq;
    auto fetch = [&](int cc, int lane) {
        const int jp = lane >> 2, pv = lane & 3;
        const uint32_t rows = (uint32_t)max(0, min(Q, p.L - cc * Q));
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xhead + (int64_t)cc * Q * p.x_sl, rows * xrow);
        const uint32_t off0 = (uint32_t)(2 * jp) * xrow + pv * 16;
#pragma unroll
        for (int m = 0; m < XPT; ++m) {
            xq[m][0] = buf_ld16_nt(rx, off0, (uint32_t)(32 * m) * xrow);
            xq[m][1] = buf_ld16_nt(rx, off0, (uint32_t)(32 * m + 1) * xrow);
        }
        const __amdgpu_buffer_rsrc_t rd =
            buf_rsrc(dthead + (int64_t)cc * Q * p.dt_sl, rows * (uint32_t)p.dt_sl * 4u);
        dtq = lane < Q ? buf_ld4(rd, lane * (uint32_t)p.dt_sl * 4u) : 0.f;
    };

    // chunk cc's output tiles from the wave's LDS scratch: four lanes cover a
    // row's 64 bytes, a store instruction 16 whole rows (storing straight from
    // the MFMA layout, every instruction would touch 32 rows).  Rows past the
    // sequence end are dropped by the buffer.
    auto store_tiles = [&](int cc, int lane) {
        const uint32_t rows = (uint32_t)min(Q, p.L - cc * Q);
        const __amdgpu_buffer_rsrc_t ry = buf_rsrc(yhead + (int64_t)cc * Q * p.y_sl, rows * (uint32_t)p.y_sl * 2u);
#pragma unroll
        for (int it = 0; it < T; ++it)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int row = (lane >> 2) + 16 * t, pc = (lane & 3) * 8;
                const uint2 lo = *(const uint2*)&s_io[wave][it][row][(lane & 3) * 4];
                const uint2 hi = *(const uint2*)&s_io[wave][it][row][16 + (lane & 3) * 4];
                const uint4 v = make_uint4(lo.x, lo.y, hi.x, hi.y);
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(decltype(__builtin_amdgcn_raw_buffer_load_b128(ry, 0, 0, 0)), v), ry,
                    ((uint32_t)(it * 32 + row) * (uint32_t)p.y_sl + pc) * 2u, 0, 0);
            }
    };

    stage(0, s_fragA, lane0);
    fetch(0, lane0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t pf = 0u, pf_sink = 0u;
    float lphi = 0.f;  // log2 of the state's pending factor: h = 2^lphi * hacc

    // chunk c, its fragments in `cur`; chunk c + 1's go to `nxt`
    auto chunk = [&](int c, bf16_t (&cur)[NF][512], bf16_t (&nxt)[NF][512]) __attribute__((always_inline)) {
        const bf16_t* F0 = &cur[0][0];
        pf_sink += pf;
        // the lane index as an opaque value: the many per-lane LDS addresses
        // below are loop-invariant, and hoisted out of the chunk loop they
        // would hold ~60 registers; recomputed here they cost a few adds
        int lane = lane0;
        asm volatile("" : "+v"(lane));
        const int r = lane & 31, half = lane >> 5;
        // ---- chunk c + 1's fragments into the other buffer (free since the
        // last barrier)
        if (c + 1 < p.nch) stage(c + 1, nxt, lane);
        // ---- the previous chunk's outputs: issued here, they have this whole
        // chunk to complete before the barrier's wait
        if (c > 0) store_tiles(c - 1, lane);
        // ---- K1: dt and its cumsum (log2 units), one position per lane
        const float cs2 = wave_incl_scan(dtq * A2);
        if (lane < Q) {
            s_cs[wave][lane] = cs2;
            s_dt[wave][lane] = dtq;
        }
        float cse[T];  // block ends, wave-uniform
#pragma unroll
        for (int k = 0; k < T; ++k)
            cse[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cs2), 32 * k + 31));
        // lazy decay (wave-uniform): phi after block k (log2), whether block k
        // applies it to the registers first (event) and by what factor
        const float lphi_in = lphi;
        float lph[T], rho[T];
        bool ev[T];
#pragma unroll
        for (int k = 0; k < T; ++k) {
            const float lk = lphi + (cse[k] - (k ? cse[k - 1] : 0.f));
            ev[k] = lk < -kLazy;
            rho[k] = __builtin_amdgcn_exp2f(lk);
            lphi = ev[k] ? 0.f : lk;
            lph[k] = lphi;
        }
        // ---- block-scaled x -> s_xg[wave][p][j] (time-major)
        const int jp = lane >> 2, pv = lane & 3;
#pragma unroll
        for (int m = 0; m < XPT; ++m) {
            const int j0 = 2 * (jp + 16 * m);
            const float ce = cse[m] - lph[m];  // rows j0, j0 + 1 sit in block m; xg / phi
            const float g0 = __shfl(dtq, j0, 64) * __builtin_amdgcn_exp2f(ce - __shfl(cs2, j0, 64));
            const float g1 = __shfl(dtq, j0 + 1, 64) * __builtin_amdgcn_exp2f(ce - __shfl(cs2, j0 + 1, 64));
            const uint32_t a0[4] = {xq[m][0].x, xq[m][0].y, xq[m][0].z, xq[m][0].w};
            const uint32_t a1[4] = {xq[m][1].x, xq[m][1].y, xq[m][1].z, xq[m][1].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                *(uint32_t*)&s_xg[wave][pv * 8 + 2 * k][j0] =
                    pack_bf16x2(__uint_as_float(a0[k] << 16) * g0, __uint_as_float(a1[k] << 16) * g1);
                *(uint32_t*)&s_xg[wave][pv * 8 + 2 * k + 1][j0] =
                    pack_bf16x2(__uint_as_float(a0[k] & 0xffff0000u) * g0,
                                __uint_as_float(a1[k] & 0xffff0000u) * g1);
            }
            // the raw rows, time-major, for D x
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                *(uint2*)&s_io[wave][m][2 * jp + e][pv * 4] = make_uint2(xq[m][e].x, xq[m][e].y);
                *(uint2*)&s_io[wave][m][2 * jp + e][16 + pv * 4] = make_uint2(xq[m][e].z, xq[m][e].w);
            }
        }
        // ---- chunk c + 1's x rows and dt into registers (they land during
        // this chunk's MFMA work)
        if (c + 1 < p.nch) fetch(c + 1, lane);
        // L2 warm-up of chunk c + 2's fragments: the workgroups of a group
        // share them and sit on one XCD; one dword per 128-byte line, spread
        // over the workgroups of the group
        if (MAMBA_SSD2_L2_WARM && c + 2 < p.nch) {
            const int nslice = (hpg / HPW) * 2, slice = (hq % (hpg / HPW)) * 2 + ph;
            const int line = threadIdx.x * nslice + slice;  // 128-byte lines of the NF KB block
            if (line < NF * 8)
                pf = *(const uint32_t*)((const char*)(gfrag + (int64_t)(c + 2) * grp_stride) + line * 128);
        }

        const uint32_t rows_c = (uint32_t)min(Q, p.L - c * Q);
        // ---- K2 + K5: y^T for the chunk's row tiles.  Inter-chunk term
        // h_in . C_i^T first, for every tile, with A from the state registers
        // (each step's C fragments are read one step ahead, so the LDS
        // latency of a read overlaps the previous step's MFMAs)
        f32x16_t yacc[T];
#pragma unroll
        for (int it = 0; it < T; ++it) yacc[it] = zero16();
        // the entering state as bf16 A operands, once: the y tiles and the
        // rare steep path read it after the state update below has moved on
        bf16x8_t hpk[NK];
#pragma unroll
        for (int kn = 0; kn < NK; ++kn) {
            float hv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = hacc[kn >> 1][8 * (kn & 1) + e];
            hpk[kn] = pack8(hv);
        }
        bf16x8_t cnext[T];
#pragma unroll
        for (int it = 0; it < T; ++it) cnext[it] = *(const bf16x8_t*)(F0 + ((FL::C0 + it * NK) * 64 + lane) * 8);
#pragma unroll
        for (int kn = 0; kn < NK; ++kn) {
            bf16x8_t cop[T];
#pragma unroll
            for (int it = 0; it < T; ++it) {
                cop[it] = cnext[it];
                if (kn + 1 < NK) cnext[it] = *(const bf16x8_t*)(F0 + ((FL::C0 + it * NK + kn + 1) * 64 + lane) * 8);
            }
#pragma unroll
            for (int it = 0; it < T; ++it) yacc[it] = mfma32x32x16(hpk[kn], cop[it], yacc[it]);
        }
        // ---- every tile as if no block were steep, the tiles' chains side by
        // side: block jt's xg operands serve all tiles it >= jt
        //   acc_it <- acc_it + S_jt / phi_jt   (jt = it: the diagonal C.B^T
        //   block, its upper triangle stored as 0 by the prep)
#pragma unroll
        for (int jt = 0; jt < T; ++jt) {
            if (ev[jt]) {
#pragma unroll
                for (int it = jt; it < T; ++it)
#pragma unroll
                    for (int v = 0; v < 16; ++v) yacc[it][v] *= rho[jt];
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int ks = 2 * jt + kk;
                const bf16x8_t a = *(const bf16x8_t*)&s_xg[wave][r][ks * 16 + 8 * half];
#pragma unroll
                for (int it = jt; it < T; ++it)
                    yacc[it] = mfma32x32x16(
                        a, *(const bf16x8_t*)(F0 + ((it * (it + 1) + ks) * 64 + lane) * 8), yacc[it]);
            }
        }
        // ---- K3 + K4 (issued before the y tiles' epilogue, whose VALU work
        // can then run beside these MFMAs): h-hat^T <- h-hat^T + B_k^T . (xg_k / phi_k) over the
        // blocks (phi applied on events only; each k step's operands read one
        // step ahead)
        bf16x8_t bnext[NTN], xnext = *(const bf16x8_t*)&s_xg[wave][r][8 * half];
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) bnext[nt] = *(const bf16x8_t*)(F0 + ((FL::B0 + nt * KS) * 64 + lane) * 8);
#pragma unroll
        for (int jt = 0; jt < T; ++jt) {
            if (ev[jt]) {
#pragma unroll
                for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
                    for (int v = 0; v < 16; ++v) hacc[nt][v] *= rho[jt];
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int ks = 2 * jt + kk;
                const bf16x8_t bx = xnext;
                bf16x8_t bop[NTN];
#pragma unroll
                for (int nt = 0; nt < NTN; ++nt) bop[nt] = bnext[nt];
                if (ks + 1 < KS) {
                    xnext = *(const bf16x8_t*)&s_xg[wave][r][(ks + 1) * 16 + 8 * half];
#pragma unroll
                    for (int nt = 0; nt < NTN; ++nt)
                        bnext[nt] = *(const bf16x8_t*)(F0 + ((FL::B0 + nt * KS + ks + 1) * 64 + lane) * 8);
                }
#pragma unroll
                for (int nt = 0; nt < NTN; ++nt) hacc[nt] = mfma32x32x16(bop[nt], bx, hacc[nt]);
            }
        }
        // y_i = exp(cs_i - cs_{e_it}) phi_it acc + D x_i, x_i raw from the chunk's
        // time-major rows; the output overwrites them in place (the same lane
        // reads and writes its 32 bytes of the row, accumulator order)
#pragma unroll
        for (int it = 0; it < T; ++it) {
            const float colf = __builtin_amdgcn_exp2f(s_cs[wave][it * 32 + r] - cse[it] + lph[it]);
            bf16_t* io = &s_io[wave][it][r][16 * half];
            const uint4 xa = *(const uint4*)io, xb = *(const uint4*)(io + 8);
            const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            uint32_t ow[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                ow[k] = pack_bf16x2(yacc[it][2 * k] * colf + Dh * __uint_as_float(xw[k] << 16),
                                    yacc[it][2 * k + 1] * colf + Dh * __uint_as_float(xw[k] & 0xffff0000u));
            *(uint4*)io = make_uint4(ow[0], ow[1], ow[2], ow[3]);
            *(uint4*)(io + 8) = make_uint4(ow[4], ow[5], ow[6], ow[7]);
        }
        // ---- steep diagonal blocks (decay beyond 2^-64 inside the block: the
        // factor exp(cs_i - cs_{e_it}) above may overflow) are recomputed: acc
        // from the state again, brought to position i (factor <= 1), then the
        // exact weights dt_j exp(cs_i - cs_j) (+ D on the diagonal) on raw x
        // rows read back from global memory
        bool steep = false;
#pragma unroll
        for (int it = 0; it < T; ++it) steep |= (it ? cse[it - 1] : 0.f) - cse[it] > kSteep;
        if (steep) {
            // block end by a wave-uniform index, as selects (no indexed registers)
            auto cse_at = [&](int k) {
                float v = cse[0];
#pragma unroll
                for (int q = 1; q < T; ++q) v = k == q ? cse[q] : v;
                return v;
            };
            auto lph_at = [&](int k) {
                float v = lph[0];
#pragma unroll
                for (int q = 1; q < T; ++q) v = k == q ? lph[q] : v;
                return v;
            };
#pragma unroll 1
            for (int it = 0; it < T; ++it) {
                const float cse_prev = it ? cse_at(it - 1) : 0.f;
                if (cse_prev - cse_at(it) <= kSteep) continue;
                const int il = it * 32 + r;
                // true units here: acc = C_i.h_in = phi_in C_i.h-hat_in, and
                // each lower block's S_k / phi_k times phi_k
                f32x16_t acc = zero16();
#pragma unroll
                for (int kn = 0; kn < NK; ++kn)
                    acc = mfma32x32x16(hpk[kn], *(const bf16x8_t*)(F0 + ((FL::C0 + it * NK + kn) * 64 + lane) * 8),
                                       acc);
                const float phin = __builtin_amdgcn_exp2f(lphi_in);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[v] *= phin;
#pragma unroll 1
                for (int jt = 0; jt < it; ++jt) {
                    const float F = __builtin_amdgcn_exp2f(cse_at(jt) - (jt ? cse_at(jt - 1) : 0.f));
                    const float ph = __builtin_amdgcn_exp2f(lph_at(jt));
                    f32x16_t t = zero16();
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) {
                        const int ks = 2 * jt + kk;
                        t = mfma32x32x16(*(const bf16x8_t*)&s_xg[wave][r][ks * 16 + 8 * half],
                                         *(const bf16x8_t*)(F0 + ((it * (it + 1) + ks) * 64 + lane) * 8), t);
                    }
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[v] = acc[v] * F + t[v] * ph;
                }
                const __amdgpu_buffer_rsrc_t rxc = buf_rsrc(xhead + (int64_t)c * Q * p.x_sl, rows_c * xrow);
                const float cs2_i = s_cs[wave][il];
                const float sc = __builtin_amdgcn_exp2f(cs2_i - cse_prev);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[v] *= sc;
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int j0 = it * 32 + kk * 16 + 8 * half;
                    float cbv[8];
                    unpack8(*(const uint4*)(F0 + ((it * (it + 1) + 2 * it + kk) * 64 + lane) * 8), cbv);
                    float m[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int j = j0 + e;
                        const float val = cbv[e] * s_dt[wave][j] * __builtin_amdgcn_exp2f(cs2_i - s_cs[wave][j]);
                        m[e] = (j < il) ? val : ((j == il) ? val + Dh : 0.f);
                    }
                    // A operand x^T[p][j0 .. j0 + 7] for p = r, from the raw rows
                    uint32_t xw[4];
#pragma unroll
                    for (int e2 = 0; e2 < 4; ++e2) {
                        const uint32_t lo = buf_ld2(rxc, ((uint32_t)(j0 + 2 * e2) * (uint32_t)p.x_sl + r) * 2u);
                        const uint32_t hi = buf_ld2(rxc, ((uint32_t)(j0 + 2 * e2 + 1) * (uint32_t)p.x_sl + r) * 2u);
                        xw[e2] = lo | (hi << 16);
                    }
                    acc = mfma32x32x16(as_bf16x8(make_uint4(xw[0], xw[1], xw[2], xw[3])), pack8(m), acc);
                }
                uint32_t ow[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) ow[k] = pack_bf16x2(acc[2 * k], acc[2 * k + 1]);
                bf16_t* io = &s_io[wave][it][r][16 * half];
                *(uint4*)io = make_uint4(ow[0], ow[1], ow[2], ow[3]);
                *(uint4*)(io + 8) = make_uint4(ow[4], ow[5], ow[6], ow[7]);
            }
        }

        // ---- this wave's loads done (chunk c + 1's fragments and x), then
        // the chunk's barrier: every wave's fragments for c + 1 have landed and
        // every wave is done with chunk c's buffer
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    for (int c = 0; c < p.nch; c += 2) {
        chunk(c, s_fragA, s_fragB);
        if (c + 1 < p.nch) chunk(c + 1, s_fragB, s_fragA);
    }
    store_tiles(p.nch - 1, lane0);
    // keeps the L2 warm-up loads alive (the condition never holds: L >= 1)
    if (p.L < 0 && pf_sink == 0x9e3779b9u) p.hT[0] = 0.f;
    // final state (f32): h[p = p0 + r][n] = phi h-hat^T[n][p]
    {
        const int r = lane0 & 31, half = lane0 >> 5;
        const float ph = __builtin_amdgcn_exp2f(lphi);
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) hacc[nt][v] *= ph;
        float* hTr = p.hT + (((int64_t)b * p.H + h) * 64 + p0 + r) * N;
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(float4*)(hTr + 32 * nt + 8 * q + 4 * half) =
                    make_float4(hacc[nt][4 * q], hacc[nt][4 * q + 1], hacc[nt][4 * q + 2], hacc[nt][4 * q + 3]);
    }
}

// ------------------------------------------------------------ host side --
static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

bool ssd2_mfma_supported(const Ssd2Params& p) {
    if (p.io_dtype != MAMBA_BF16) return false;
    if (p.P != 64 || (p.N != 64 && p.N != 128)) return false;
    if (p.Q % 32 != 0 || p.Q > kMaxQ) return false;
    if (!aligned16(p.x) || !aligned16(p.Bm) || !aligned16(p.Cm) || !aligned16(p.y)) return false;
    const int64_t s[] = {p.x_sb, p.x_sl, p.x_sh, p.B_sb, p.B_sl, p.B_sg, p.C_sb, p.C_sl, p.C_sg};
    for (int64_t v : s)
        if (v % 8 != 0) return false;
    // x and y rows are addressed through 32-bit buffer offsets inside one
    // chunk, and a row must hold the whole headdim
    if (p.x_sl < p.P || p.y_sl < p.P || p.dt_sl < 1 || (int64_t)p.Q * p.x_sl * 2 >= (1ll << 31) ||
        (int64_t)p.Q * p.y_sl * 2 >= (1ll << 31) || (int64_t)p.Q * p.dt_sl * 4 >= (1ll << 31))
        return false;
    return true;
}

// The MFMA path chunks at min(chunk_len, 64) positions, a chunk's positions
// being a wave's lanes: the chunked form is exact for any chunk length, so
// only rounding differs.
constexpr int kFastQ = 64;

static Ssd2Params fast_params(const Ssd2Params& p) {
    Ssd2Params q = p;
    q.Q = p.Q < kFastQ ? p.Q : kFastQ;
    q.nch = (p.L + q.Q - 1) / q.Q;
    return q;
}

static size_t frag_count(const Ssd2Params& p) {
    const int T = p.Q / 32, NK = p.N / 16, KS = p.Q / 16, NTN = p.N / 32;
    return (size_t)(T * (T + 1) + T * NK + NTN * KS);
}

size_t ssd2_mfma_workspace(const Ssd2Params& p0) {
    const Ssd2Params p = fast_params(p0);
    return align_up((size_t)p.nb * p.nch * p.G * frag_count(p) * 1024, 256);
}

// Heads per workgroup (waves per workgroup): one of 5, 4, 2, 1 dividing the
// heads of a group.  The scan kernel's LDS (two chunks of group fragments)
// allows one workgroup per CU, so a launch of nwg workgroups takes
// ceil(nwg / 256) rounds on MI355X's 256 CUs, each as long as the busiest
// SIMD's ceil(HPW / 4) waves.  Ties go to the larger set, which stages each
// fragment for more heads.  MAMBA_SSD2_HPW (read on every call) forces a
// valid choice.
static int choose_hpw(const Ssd2Params& p) {
    const int hpg = p.H / p.G;
    const char* e = getenv("MAMBA_SSD2_HPW");
    if (e) {
        const int v = atoi(e);
        if ((v == 1 || v == 2 || v == 4 || v == 5) && hpg % v == 0) return v;
    }
    constexpr int kCUs = 256;
    int best = 1;
    int64_t best_cost = INT64_MAX;
    for (int hpw : {5, 4, 2, 1}) {
        if (hpg % hpw != 0) continue;
        const int64_t nwg = (int64_t)p.nb * (p.H / hpw) * 2;
        const int64_t cost = (nwg + kCUs - 1) / kCUs * ((hpw + 3) / 4);
        if (cost < best_cost) {
            best_cost = cost;
            best = hpw;
        }
    }
    return best;
}

template <int N, int Q, int HPW>
static void launch_scan(const Ssd2Params& p, const bf16_t* frag, hipStream_t stream) {
    const int nwg = p.nb * (p.H / HPW) * 2;
    hipLaunchKernelGGL((ssd2_scan_wu<N, Q, HPW>), dim3(nwg), dim3(64 * HPW), 0, stream, p, frag);
}

template <int N, int Q>
static int launch_q(const Ssd2Params& p, void* ws, hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    bf16_t* frag = (bf16_t*)ws;
    hipLaunchKernelGGL((ssd2_prep_pack<N, Q>), dim3(p.nch * p.G, p.nb), dim3(256), 0, stream, p, frag);
    MAMBA_CHECK_LAUNCH();
    if (ev0) MAMBA_CHECK_HIP(hipEventRecord(ev0, stream));
    switch (choose_hpw(p)) {
        case 5: launch_scan<N, Q, 5>(p, frag, stream); break;
        case 4: launch_scan<N, Q, 4>(p, frag, stream); break;
        case 2: launch_scan<N, Q, 2>(p, frag, stream); break;
        default: launch_scan<N, Q, 1>(p, frag, stream); break;
    }
    MAMBA_CHECK_LAUNCH();
    if (ev1) MAMBA_CHECK_HIP(hipEventRecord(ev1, stream));
    return MAMBA_OK;
}

int ssd2_mfma_launch(const Ssd2Params& p0, void* ws, hipStream_t stream, hipEvent_t ev0, hipEvent_t ev1) {
    const Ssd2Params p = fast_params(p0);
    if (p.N == 64)
        return p.Q == 32 ? launch_q<64, 32>(p, ws, stream, ev0, ev1) : launch_q<64, 64>(p, ws, stream, ev0, ev1);
    return p.Q == 32 ? launch_q<128, 32>(p, ws, stream, ev0, ev1) : launch_q<128, 64>(p, ws, stream, ev0, ev1);
}

int ssd2_mfma_hpw(const Ssd2Params& p) { return choose_hpw(fast_params(p)); }

}  // namespace mamba
