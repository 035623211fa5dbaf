// Mamba-3 prefill around the single-SSD seam, gfx950: the prologue that turns
// the in_proj output into the seam's inputs, and the epilogue after it.
//
// Reference: Mamba3::forward_single_ssd (burn-mamba
// src/mamba3/single_ssd/single_ssd/mod.rs:44-360).
//  * mamba3_prep_fwd (steps 2-6, :86-262): trapezoidal_coefficients
//    (helpers.rs:42-73); scale_t = gamma_t + (1 - lambda_{t+1}) dt_{t+1}
//    (:129-150); qk_norm_expand_bias (helpers.rs:82-95); rotate_bc_forward
//    Complex2D (rotation/mod.rs:653-679: cumulative angle prev +
//    cumsum_s(dt range pi tanh(rot)), apply_rope_partial rope.rs:118-170);
//    v = x mimo_x (helpers.rs:152-168); the beta seed
//    h0 = ssm + (dt_0 - gamma_0) sum_m (v_prev mimo_x[m]) (x) K_prev[m]
//    (:195-225); the cache tail (last token's rotated B and x, wrapped angle;
//    the angle goes to a separate buffer because every (b, h, m) workgroup
//    reads the starting angle).
//  * mamba3_finish_fwd (step 9 before out_proj, :288-332): y += D v, the silu
//    gate (or per-head gated RMSNorm) with mimo_z, and the mimo_o merge.
// The cumulative angle is carried on a fixed-point grid (2^-32 rad, reduced
// modulo 2 pi): the same cos / sin as the reference's unwrapped f32 cumsum,
// without its drift on long sequences, and the same value at every position
// whatever the kernel's segmentation.
#include "mamba3_internal.h"

namespace mamba {

__device__ __forceinline__ float m3p_ld(const M3PrepParams& p, int b, int l, int i) {
    const int64_t off = (int64_t)b * p.proj_sb + (int64_t)l * p.proj_sl + i;
    return p.proj_bf16 ? bf16_to_f32(static_cast<const bf16_t*>(p.proj)[off]) : static_cast<const float*>(p.proj)[off];
}
__device__ __forceinline__ void m3p_st(bool bf, void* base, int64_t i, float v) {
    if (bf)
        static_cast<bf16_t*>(base)[i] = f32_to_bf16(v);
    else
        static_cast<float*>(base)[i] = v;
}

// dt, lambda of (b, l, h); l past the end gives dt = lambda = 0 (scale's shift)
__device__ __forceinline__ void m3p_coef(const M3PrepParams& p, int b, int l, int h, float& dt, float& da,
                                         float& lam) {
    if (l >= p.L) {
        dt = da = lam = 0.f;
        return;
    }
    const int o = 2 * p.H * p.P + 2 * p.M * p.G * p.N;
    m3_coef(m3p_ld(p, b, l, o + h), m3p_ld(p, b, l, o + p.H + h), m3p_ld(p, b, l, o + 2 * p.H + h), p.dt_bias[h],
            p.a_floor, p.dt_lo, p.dt_hi, dt, da, lam);
}

// Beta seed of the initial state: reads the previous token's K / v_state
// before the prep kernels replace them.  Grid (b * H, row blocks): a
// workgroup seeds rows_per rows of one (b, h) state, with v_state mimo_x and
// K staged in LDS and its (at most kSeedE) state loads per thread issued
// before the first is used.  Dynamic LDS: [M][rows_per] + [M][N] floats.
constexpr int kSeedE = 8;
__global__ __launch_bounds__(256) void mamba3_seed_kernel(M3PrepParams p, int rows_per) {
    extern __shared__ float s_seed[];
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H, t = threadIdx.x;
    const int p0 = blockIdx.y * rows_per, nr = min(rows_per, p.P - p0);
    if (nr <= 0) return;  // uniform over the workgroup
    float* s_vx = s_seed;                  // [M][rows_per]
    float* s_k = s_seed + p.M * rows_per;  // [M][N]
    const int64_t bh = (int64_t)b * p.H + h;
    const int64_t base = bh * p.P * p.N + (int64_t)p0 * p.N;
    const int ne = nr * p.N;
    float hv[kSeedE];
#pragma unroll
    for (int j = 0; j < kSeedE; ++j) {
        const int e = t + 256 * j;
        hv[j] = e < ne ? p.ssm[base + e] : 0.f;
    }
    for (int i = t; i < p.M * nr; i += 256) {
        const int m = i / nr, r = i % nr;
        const float mxv = p.mx ? p.mx[((int64_t)h * p.M + m) * p.P + p0 + r] : 1.f;
        s_vx[m * rows_per + r] = p.vst[bh * p.P + p0 + r] * mxv;
    }
    for (int i = t; i < p.M * p.N; i += 256) {
        const int m = i / p.N, n = i % p.N;
        s_k[i] = p.kst[(((int64_t)b * p.M + m) * p.H + h) * p.N + n];
    }
    float dt, da, lam;
    m3p_coef(p, b, 0, h, dt, da, lam);
    const float f = dt - lam * dt;  // dt_0 - gamma_0
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSeedE; ++j) {
        const int e = t + 256 * j;
        if (e < ne) {
            const int r = e / p.N, n = e % p.N;
            float acc = 0.f;
            for (int m = 0; m < p.M; ++m) acc += s_vx[m * rows_per + r] * s_k[m * p.N + n];
            p.h0[base + e] = hv[j] + f * acc;
        }
    }
}

// One workgroup per (b, h, m): positions in tiles of TS; the angle scan of
// (b, h) is carried by threads a < A (recomputed by every m of the head).
// N (dstate, a power of two) is a template parameter so the per-element loops
// are (row, column) walks with shifts, not runtime divisions.
template <int TS, int N>
__global__ __launch_bounds__(256) void mamba3_prep_kernel(M3PrepParams p) {
    constexpr int RS = N >= 256 ? 1 : 256 / N;  // rows per pass of a [rows][N] walk
    const int m = blockIdx.x % p.M, h = (blockIdx.x / p.M) % p.H, b = blockIdx.x / (p.M * p.H);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int P = p.P, g = h / (p.H / p.G);
    const int col = t % N, row0 = t / N;  // N <= 256: every thread owns one column
    const int64_t bh = (int64_t)b * p.H + h;
    const int d_inner = p.H * P, bc = p.M * p.G * N;
    const int o_b = 2 * d_inner + (m * p.G + g) * N, o_c = o_b + bc;
    const int o_rot = 2 * d_inner + 2 * bc + 3 * p.H;
    const int npair = p.R / 2, A = p.A;
    extern __shared__ __align__(16) float s_dyn[];
    float* s_raw = s_dyn;                  // [2 TS][N]: B rows, then C rows
    float* s_cs = s_raw + 2 * TS * N;      // [TS][npair]
    float* s_sn = s_cs + TS * npair;       // [TS][npair]
    float* s_th = s_sn + TS * npair;       // [TS][A]: angle increments, then cumulative angles
    float* s_x = s_th + TS * A;            // [TS][P]: x rows of the tile
    __shared__ float s_dt[TS + 1], s_lam[TS + 1], s_da[TS], s_rms[2 * TS];
    const float bnw = p.bnw[col], cnw = p.cnw[col];
    const float bbias = p.bbias[((int64_t)h * p.M + m) * N + col], cbias = p.cbias[((int64_t)h * p.M + m) * N + col];
    // rotation partner of this column: pairs (2k, 2k+1) for M == 1, (k, k + N/2) otherwise
    const bool pw = p.M == 1;
    const int k_of = pw ? col >> 1 : (col < N / 2 ? col : col - N / 2);
    const bool first = pw ? (col & 1) == 0 : col < N / 2;
    const int partner = pw ? (col ^ 1) : (first ? col + N / 2 : col - N / 2);
    const bool rotated = k_of < npair;
    // 2-D walks over the tile for the runtime widths A (angles), npair and P:
    // this thread's column and row offset, and the row step, computed once
    const int ca = t % A, ra0 = t / A, rsa = A >= 256 ? 1 : 256 / A;
    const int np1 = npair > 0 ? npair : 1;
    const int cp = t % np1, rp0 = t / np1, rsp = np1 >= 256 ? 1 : 256 / np1;
    const int cx = t % P, rx0 = t / P, rsx = P >= 256 ? 1 : 256 / P;

    int theta = (t < A) ? m3_ang_fix(p.ang[bh * A + t]) : 0;  // grid units
    for (int l0 = 0; l0 < p.L; l0 += TS) {
        const int nt = min(TS, p.L - l0);
        // coefficients of the tile (+ the next position for scale)
        if (t <= TS) {
            float dt, da, lam;
            m3p_coef(p, b, l0 + t, h, dt, da, lam);
            s_dt[t] = dt;
            s_lam[t] = lam;
            if (t < TS) s_da[t] = da;
        }
        // raw B/C rows of (m, g): row r < TS is B, r >= TS is C; the tile's x rows.
        // Everything the tile reads from HBM is staged here, before any global
        // store (proj and the outputs are untyped pointers the compiler must
        // assume may alias, which would serialise load -> store pairs).
        for (int r = row0; r < 2 * TS; r += RS) {
            const int rr = r < TS ? r : r - TS;
            s_raw[r * N + col] = rr < nt ? m3p_ld(p, b, l0 + rr, (r < TS ? o_b : o_c) + col) : 0.f;
        }
        if (P <= 256) {
            for (int r = rx0; r < nt; r += rsx) s_x[r * P + cx] = m3p_ld(p, b, l0 + r, d_inner + h * P + cx);
        } else {
            for (int r = 0; r < nt; ++r)
                for (int pp = t; pp < P; pp += 256) s_x[r * P + pp] = m3p_ld(p, b, l0 + r, d_inner + h * P + pp);
        }
        // raw rotation channels of the tile
        if (A <= 256) {
            for (int r = ra0; r < nt; r += rsa) s_th[r * A + ca] = m3p_ld(p, b, l0 + r, o_rot + ca);
        } else {
            for (int r = 0; r < nt; ++r)
                for (int k = t; k < A; k += 256) s_th[r * A + k] = m3p_ld(p, b, l0 + r, o_rot + k);
        }
        __syncthreads();
        // angle increments dt range pi tanh(rot), spread over all threads
        if (A <= 256) {
            for (int r = ra0; r < nt; r += rsa) s_th[r * A + ca] = m3_angle_inc(s_dt[r], s_th[r * A + ca], p.span);
        } else {
            for (int r = 0; r < nt; ++r)
                for (int k = t; k < A; k += 256) s_th[r * A + k] = m3_angle_inc(s_dt[r], s_th[r * A + k], p.span);
        }
        // QK-norm sums of squares: 2 TS rows, one wave per row (strided)
        for (int rr = wave; rr < 2 * TS; rr += 4) {
            const float* src = s_raw + rr * N;
            float ss = 0.f;
            for (int n = lane; n < N; n += 64) ss += src[n] * src[n];
            ss = wave_sum(ss);
            if (lane == 0) s_rms[rr] = m3_rms_inv(ss, N);
        }
        __syncthreads();
        // cumulative angle: sequential per angle over the tile (LDS only), on the fixed-point grid
        if (t < A)
            for (int r = 0; r < nt; ++r) {
                theta = m3_ang_reduce(theta + m3_ang_fix(s_th[r * A + t]));
                s_th[r * A + t] = m3_ang_rad(theta);
            }
        // normalise + bias in place
        for (int r = row0; r < 2 * TS; r += RS)
            s_raw[r * N + col] = m3_norm(s_raw[r * N + col], s_rms[r], r < TS ? bnw : cnw, r < TS ? bbias : cbias);
        __syncthreads();
        // cos / sin of the rotated pairs' angles, spread over all threads
        if (npair > 0 && npair <= 256) {
            for (int r = rp0; r < nt; r += rsp) {
                const float th = s_th[r * A + cp];
                s_cs[r * npair + cp] = cosf(th);
                s_sn[r * npair + cp] = sinf(th);
            }
        } else if (npair > 256) {
            for (int r = 0; r < nt; ++r)
                for (int k = t; k < npair; k += 256) {
                    s_cs[r * npair + k] = cosf(s_th[r * A + k]);
                    s_sn[r * npair + k] = sinf(s_th[r * A + k]);
                }
        }
        __syncthreads();
        // rotate and store: each thread owns column col of its rows, reading its partner
        for (int r = row0; r < 2 * TS; r += RS) {
            const int rr = r < TS ? r : r - TS;
            if (rr >= nt) continue;
            float v = s_raw[r * N + col];
            if (rotated) {
                const float cs = s_cs[rr * npair + k_of], sn = s_sn[rr * npair + k_of];
                const float o = s_raw[r * N + partner];
                v = m3_rot(cs, v, first ? -sn : sn, o);
            }
            const int64_t oi = ((((int64_t)b * p.L + l0 + rr) * p.M + m) * p.H + h) * N + col;
            m3p_st(p.io_bf16, r < TS ? p.Bo : p.Co, oi, v);
            // the cache tail: the last token's rotated B
            if (r < TS && l0 + rr == p.L - 1) p.kst[(((int64_t)b * p.M + m) * p.H + h) * N + col] = v;
        }
        // v = x mimo_x [b, l, m, h, p]; da / gamma / scale (m == 0)
        for (int pp = t; pp < P; pp += 256) {
            const float mxv = p.mx ? p.mx[((int64_t)h * p.M + m) * P + pp] : 1.f;
            for (int r = 0; r < nt; ++r) {
                const int64_t oi = ((((int64_t)b * p.L + l0 + r) * p.M + m) * p.H + h) * P + pp;
                m3p_st(p.io_bf16, p.v, oi, s_x[r * P + pp] * mxv);
            }
        }
        if (m == 0 && t < nt) {
            const int64_t o = ((int64_t)b * p.L + l0 + t) * p.H + h;
            const float gmv = s_lam[t] * s_dt[t];
            p.da[o] = s_da[t];
            p.gm[o] = gmv;
            p.sc[o] = __builtin_fmaf(1.f - s_lam[t + 1], s_dt[t + 1], gmv);
        }
        // the rest of the cache tail (m == 0): the last x and the wrapped angle
        if (l0 + nt == p.L && m == 0) {
            for (int pp = t; pp < P; pp += 256) p.vst[bh * P + pp] = s_x[(nt - 1) * P + pp];
            if (t < A) p.ang_out[bh * A + t] = m3_ang_rad(theta);
        }
        __syncthreads();  // LDS reuse by the next tile
    }
}

// ---- segment-parallel fast path -------------------------------------------
// The sequence is cut into segments of kM3Seg positions (fewer, down to one
// 32-position tile, where the launch would have under 512 (b, h, segment)
// workgroups: the angles are integer sums, so the segmentation does not change
// any result).  A first kernel sums
// each segment's angle increments dt range pi tanh(rot) per (head, angle) on
// the fixed-point angle grid; the main kernel then runs one workgroup per (b,
// h, segment) over every MIMO rank, starting from the cache's angle plus the
// earlier segments' totals, and adds the increments position by position.  Loads and
// stores of proj rows, B, C and v are 8- or 4-wide vectors; proj and the
// outputs are typed by template parameters.
constexpr int kM3Seg = 256, kM3Tile = 32;

template <typename T> __device__ __forceinline__ float m3_ld1(const T* q);
template <> __device__ __forceinline__ float m3_ld1<float>(const float* q) { return *q; }
template <> __device__ __forceinline__ float m3_ld1<bf16_t>(const bf16_t* q) { return bf16_to_f32(*q); }

// 8 consecutive elements, 16-byte aligned start
template <typename T> __device__ __forceinline__ void m3_ld8(const T* q, float* o);
template <> __device__ __forceinline__ void m3_ld8<float>(const float* q, float* o) {
    const float4 a = *(const float4*)q, c = *(const float4*)(q + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = c.x; o[5] = c.y; o[6] = c.z; o[7] = c.w;
}
template <> __device__ __forceinline__ void m3_ld8<bf16_t>(const bf16_t* q, float* o) {
    const uint4 u = *(const uint4*)q;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o[2 * k] = __uint_as_float(w[k] << 16);
        o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}
// 4 consecutive elements, aligned to their size
template <typename T> __device__ __forceinline__ void m3_ld4(const T* q, float* o);
template <> __device__ __forceinline__ void m3_ld4<float>(const float* q, float* o) {
    const float4 a = *(const float4*)q;
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
}
template <> __device__ __forceinline__ void m3_ld4<bf16_t>(const bf16_t* q, float* o) {
    const uint2 u = *(const uint2*)q;
    o[0] = __uint_as_float(u.x << 16); o[1] = __uint_as_float(u.x & 0xffff0000u);
    o[2] = __uint_as_float(u.y << 16); o[3] = __uint_as_float(u.y & 0xffff0000u);
}
// Raw 8 consecutive elements, converted where used: a group of loads is
// issued together and its elements unpacked only when consumed.
template <typename T> struct M3Raw8;
template <> struct M3Raw8<bf16_t> { uint4 u; };
template <> struct M3Raw8<float> { float4 a, c; };
__device__ __forceinline__ M3Raw8<bf16_t> m3_raw8(const bf16_t* q) { return {*(const uint4*)q}; }
__device__ __forceinline__ M3Raw8<float> m3_raw8(const float* q) {
    return {*(const float4*)q, *(const float4*)(q + 4)};
}
__device__ __forceinline__ void m3_cvt8(const M3Raw8<bf16_t>& r, float* o) {
    const uint32_t w[4] = {r.u.x, r.u.y, r.u.z, r.u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o[2 * k] = __uint_as_float(w[k] << 16);
        o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}
__device__ __forceinline__ void m3_cvt8(const M3Raw8<float>& r, float* o) {
    o[0] = r.a.x; o[1] = r.a.y; o[2] = r.a.z; o[3] = r.a.w; o[4] = r.c.x; o[5] = r.c.y; o[6] = r.c.z; o[7] = r.c.w;
}

template <typename T> __device__ __forceinline__ void m3_st8(T* q, const float* v);
template <> __device__ __forceinline__ void m3_st8<float>(float* q, const float* v) {
    *(float4*)q = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(q + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
template <> __device__ __forceinline__ void m3_st8<bf16_t>(bf16_t* q, const float* v) {
    *(uint4*)q = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                            pack_bf16x2(v[6], v[7]));
}
template <typename T> __device__ __forceinline__ void m3_st4(T* q, const float* v);
template <> __device__ __forceinline__ void m3_st4<float>(float* q, const float* v) {
    *(float4*)q = make_float4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ void m3_st4<bf16_t>(bf16_t* q, const float* v) {
    *(uint2*)q = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

template <typename TP>
__device__ __forceinline__ void m3_coef_t(const M3PrepParams& p, const TP* proj, int b, int l, int h, float& dt,
                                          float& da, float& lam) {
    if (l >= p.L) {
        dt = da = lam = 0.f;
        return;
    }
    const TP* row = proj + (int64_t)b * p.proj_sb + (int64_t)l * p.proj_sl + 2 * p.H * p.P + 2 * p.M * p.G * p.N;
    m3_coef(m3_ld1(row + h), m3_ld1(row + p.H + h), m3_ld1(row + 2 * p.H + h), p.dt_bias[h], p.a_floor, p.dt_lo,
            p.dt_hi, dt, da, lam);
}

// Per (b, segment): tot[b][seg][h][a] = sum over the segment's positions of
// dt[b, l, h] * (tanh(rot[b, l, a]) * span), each term formed exactly as the
// main kernel forms it and put on the fixed-point angle grid, the sum reduced
// modulo 2 pi on that grid.  Grid (b * nseg, head groups):
// a workgroup takes hpw heads (hpw * A <= 256 where possible, one (h, a) pair
// per thread) so that b * nseg * H / hpw workgroups share the segments.
// Dynamic LDS: [tile][hpw] dt and [tile][A] tanh(rot) * span.
template <typename TP>
__global__ __launch_bounds__(256) void mamba3_angle_tot_kernel(M3PrepParams p, int nseg, int seg_len, int hpw,
                                                               int* tot) {
    const int b = blockIdx.x / nseg, seg = blockIdx.x % nseg, t = threadIdx.x;
    const TP* proj = static_cast<const TP*>(p.proj);
    const int H = p.H, A = p.A, HA = H * A;
    const int h0 = blockIdx.y * hpw, nh = min(hpw, H - h0), np = nh * A;  // this group's pairs
    const int l_begin = seg * seg_len, l_end = min(p.L, l_begin + seg_len);
    const int o_rot = 2 * H * p.P + 2 * p.M * p.G * p.N + 3 * H;
    extern __shared__ __align__(16) float s_dyn[];
    float* s_dtt = s_dyn;                  // [kM3Tile][hpw]
    float* s_tr = s_dtt + kM3Tile * hpw;   // [kM3Tile][A]
    constexpr int KP = 4;                  // (h, a) pairs per thread and pass
    for (int pb = 0; pb < np; pb += 256 * KP) {
        int acc[KP];
#pragma unroll
        for (int k = 0; k < KP; ++k) acc[k] = 0;
        for (int l0 = l_begin; l0 < l_end; l0 += kM3Tile) {
            const int nt = min(kM3Tile, l_end - l0);
            for (int i = t; i < kM3Tile * nh; i += 256) {
                const int r = i / nh, hl = i % nh;
                float dt = 0.f, da, lam;
                if (r < nt) m3_coef_t(p, proj, b, l0 + r, h0 + hl, dt, da, lam);
                s_dtt[r * hpw + hl] = dt;
            }
            for (int i = t; i < kM3Tile * A; i += 256) {
                const int r = i / A, a = i % A;
                s_tr[i] = r < nt ? m3_ld1(proj + (int64_t)b * p.proj_sb + (int64_t)(l0 + r) * p.proj_sl + o_rot + a)
                                 : 0.f;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                const int i = pb + t + 256 * k;
                if (i < np) {
                    const int hl = i / A, a = i % A;
                    int sacc = acc[k];
                    for (int r = 0; r < nt; ++r)
                        sacc += m3_ang_fix(m3_angle_inc(s_dtt[r * hpw + hl], s_tr[r * A + a], p.span));
                    acc[k] = m3_ang_reduce(sacc);
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int i = pb + t + 256 * k;
            if (i < np) tot[((int64_t)b * nseg + seg) * HA + (int64_t)h0 * A + i] = acc[k];
        }
    }
}

// One workgroup per (b, h, segment), every MIMO rank.  Dynamic LDS: the
// angle increments / cumulative angles [kM3Tile][A4] (A4 = A rounded up to 4)
// and cos / sin tables [kM3Tile][N/2] over every pair index k, with the
// identity (1, 0) for the pairs past the rotated ones, so a thread reads its
// columns' factors as aligned vectors and rotates without selects.  When 2 M
// divides the rows of a pass (256 / (N / 8)), every thread keeps one (B or C,
// rank) and its column block for the whole segment; otherwise the rows are
// decomposed per pass.
template <typename TP, typename TO, int N>
__global__ __launch_bounds__(256) void mamba3_prep_seg_kernel(M3PrepParams p, int nseg, int seg_len, const int* tot) {
    constexpr int TPR = N / 8;         // threads per B/C row (8 columns each)
    constexpr int RPP = 256 / TPR;     // rows per pass
    constexpr int W = N / 2;           // pair indices
    const int seg = blockIdx.x % nseg, h = (blockIdx.x / nseg) % p.H, b = blockIdx.x / (nseg * p.H);
    const int t = threadIdx.x;
    const TP* proj = static_cast<const TP*>(p.proj);
    const int P = p.P, M = p.M, A = p.A, A4 = (p.A + 3) & ~3, npair = p.R / 2, g = h / (p.H / p.G);
    const int d_inner = p.H * P, bc = M * p.G * N;
    const int o_rot = 2 * d_inner + 2 * bc + 3 * p.H;
    const int64_t bh = (int64_t)b * p.H + h;
    const int l_begin = seg * seg_len, l_end = min(p.L, l_begin + seg_len);
    const TP* projb = proj + (int64_t)b * p.proj_sb;
    extern __shared__ __align__(16) float s_dyn[];
    float* s_th = s_dyn;                   // [kM3Tile][A4]
    float* s_cs = s_th + kM3Tile * A4;     // [kM3Tile][W]
    float* s_sn = s_cs + kM3Tile * W;      // [kM3Tile][W]
    __shared__ float s_dt[kM3Tile + 1], s_lam[kM3Tile + 1], s_da[kM3Tile];

    // starting angle of the segment (grid units): the cache's angle plus the earlier segments' totals
    int theta = 0;
    if (t < A) {
        theta = m3_ang_fix(p.ang[bh * A + t]);
        for (int s2 = 0; s2 < seg; ++s2)
            theta = m3_ang_reduce(theta + tot[((int64_t)b * nseg + s2) * p.H * A + (int64_t)h * A + t]);
    }
    // this thread's 8 columns of every B/C row, their pair indices and rotation sign
    const int col0 = (t % TPR) * 8, rsub = t / TPR;
    const bool pairwise = M == 1;            // pairs (2k, 2k+1); else (k, k + N/2)
    const int kbase = pairwise ? col0 / 2 : (TPR == 1 ? 0 : (col0 < N / 2 ? col0 : col0 - N / 2));
    const float sgn = col0 < N / 2 ? -1.f : 1.f;  // y' = c y + sgn s y_partner (M > 1)
    const bool fixed = RPP % (2 * M) == 0;   // one (B or C, rank) per thread
    const int which_f = (rsub % (2 * M)) / M, m_f = rsub % M, dpos = RPP / (2 * M);
    float w8[8], bias8[8];
    if (fixed) {
        const float* wsrc = which_f ? p.cnw : p.bnw;
        const float* bsrc = (which_f ? p.cbias : p.bbias) + ((int64_t)h * M + m_f) * N + col0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            w8[e] = wsrc[col0 + e];
            bias8[e] = bsrc[e];
        }
    }

    const int PQ = P / 4;
    const bool vfixed = 256 % (M * PQ) == 0;
    const int vpq = t % PQ, vm = (t / PQ) % M, vr0 = t / (M * PQ), vdr = vfixed ? 256 / (M * PQ) : 1;
    float4 vmx = make_float4(1.f, 1.f, 1.f, 1.f);
    if (vfixed && p.mx) vmx = *(const float4*)(p.mx + ((int64_t)h * M + vm) * P + 4 * vpq);

    // one B/C row: norm, weight, bias, rotation, store (and the cache tail)
    auto bc_src = [&](int l, int which, int m) {
        return projb + (int64_t)l * p.proj_sl + 2 * d_inner + which * bc + (m * p.G + g) * N + col0;
    };
    auto bc_finish = [&](int l0, int r, int which, int m, const float* w, const float* bias, float* y) {
        const int l = l0 + r;
        float ss = m3_sumsq8(y);
        ss = m3_group_sum<TPR>(ss);
        const float rms = m3_rms_inv(ss, N);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = m3_norm(y[e], rms, w[e], bias[e]);
        const float* csr = (const float*)__builtin_assume_aligned(s_cs + r * W + kbase, 16);
        const float* snr = (const float*)__builtin_assume_aligned(s_sn + r * W + kbase, 16);
        if (pairwise) {
            const float4 c4 = *(const float4*)csr, s4 = *(const float4*)snr;
            const float cv[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float y0 = y[2 * j], y1 = y[2 * j + 1];
                y[2 * j] = m3_rot(cv[j], y0, -sv[j], y1);
                y[2 * j + 1] = m3_rot(cv[j], y1, sv[j], y0);
            }
        } else if (TPR == 1) {  // N == 8: the pairs (k, k + 4) are both in this thread
            const float4 c4 = *(const float4*)csr, s4 = *(const float4*)snr;
            const float cv[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float y0 = y[j], y1 = y[j + 4];
                y[j] = m3_rot(cv[j], y0, -sv[j], y1);
                y[j + 4] = m3_rot(cv[j], y1, sv[j], y0);
            }
        } else {
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = m3_xor<TPR / 2>(y[e]);
            const float4 c0 = *(const float4*)csr, c1 = *(const float4*)(csr + 4);
            const float4 s0 = *(const float4*)snr, s1 = *(const float4*)(snr + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = m3_rot(cv[e], y[e], sgn * sv[e], o[e]);
        }
        const int64_t oi = ((((int64_t)b * p.L + l) * M + m) * p.H + h) * N + col0;
        m3_st8(static_cast<TO*>(which ? p.Co : p.Bo) + oi, y);
        // the cache tail: the last token's rotated B
        if (!which && l == p.L - 1) {
            float* kq = p.kst + (((int64_t)b * M + m) * p.H + h) * N + col0;
            *(float4*)kq = make_float4(y[0], y[1], y[2], y[3]);
            *(float4*)(kq + 4) = make_float4(y[4], y[5], y[6], y[7]);
        }
    };
    auto bc_row = [&](int l0, int r, int which, int m, const float* w, const float* bias) {
        float y[8];
        m3_ld8(bc_src(l0 + r, which, m), y);
        bc_finish(l0, r, which, m, w, bias, y);
    };
    constexpr int kBCG = 2;  // B/C rows whose loads are issued together (fixed path)

    for (int l0 = l_begin; l0 < l_end; l0 += kM3Tile) {
        const int nt = min(kM3Tile, l_end - l0);
        // coefficients of the tile and of the position after it (scale's shift)
        if (t <= kM3Tile) {
            float dt = 0.f, da = 0.f, lam = 0.f;  // past the tile's next position: unused
            if (t <= nt) m3_coef_t(p, proj, b, l0 + t, h, dt, da, lam);
            s_dt[t] = dt;
            s_lam[t] = lam;
            if (t < kM3Tile) s_da[t] = da;
        }
        __syncthreads();
        // angle increments dt range pi tanh(rot)
        for (int i = t; i < nt * A; i += 256) {
            const int r = i / A, a = i - r * A;
            s_th[r * A4 + a] = m3_angle_inc(s_dt[r], m3_ld1(projb + (int64_t)(l0 + r) * p.proj_sl + o_rot + a), p.span);
        }
        __syncthreads();
        // cumulative angle on the fixed-point grid, in radians ([-pi, pi]) at every position
        if (t < A)
            for (int r = 0; r < nt; ++r) {
                theta = m3_ang_reduce(theta + m3_ang_fix(s_th[r * A4 + t]));
                s_th[r * A4 + t] = m3_ang_rad(theta);
            }
        __syncthreads();
        // cos / sin of the wrapped angles (|angle| <= pi); identity past the rotated pairs
        for (int i = t; i < nt * W; i += 256) {
            const int r = i / W, k = i % W;
            float c = 1.f, sn = 0.f;
            if (k < npair) m3_cossin(s_th[r * A4 + k], c, sn);
            s_cs[i] = c;
            s_sn[i] = sn;
        }
        __syncthreads();
        // B / C rows
        if (fixed) {
            // kBCG rows per group, their loads issued before the first is used (rows
            // clamped into the tile so that the loads are unconditional)
            for (int r0 = rsub / (2 * M); r0 < nt; r0 += kBCG * dpos) {
                M3Raw8<TP> q[kBCG];
#pragma unroll
                for (int j = 0; j < kBCG; ++j) q[j] = m3_raw8(bc_src(l0 + min(r0 + j * dpos, nt - 1), which_f, m_f));
#pragma unroll
                for (int j = 0; j < kBCG; ++j) {
                    if (r0 + j * dpos < nt) {
                        float y[8];
                        m3_cvt8(q[j], y);
                        bc_finish(l0, r0 + j * dpos, which_f, m_f, w8, bias8, y);
                    }
                }
            }
        } else {
            for (int rb = rsub; rb < nt * 2 * M; rb += RPP) {
                const int m = rb % M, which = (rb / M) & 1, r = rb / (2 * M);
                float w[8], bias[8];
                const float* bsrc = (which ? p.cbias : p.bbias) + ((int64_t)h * M + m) * N + col0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    w[e] = (which ? p.cnw : p.bnw)[col0 + e];
                    bias[e] = bsrc[e];
                }
                bc_row(l0, r, which, m, w, bias);
            }
        }
        // v = x mimo_x [b, l, m, h, p], four headdim values per item; with
        // 256 % (M P / 4) == 0 each thread keeps one (rank, quad) of the head
        if (vfixed) {
            // kVG rows per group, their loads issued before the first is used
            constexpr int kVG = 4;
            const TP* xs = projb + d_inner + h * P + 4 * vpq;
            for (int r0 = vr0; r0 < nt; r0 += kVG * vdr) {
                float x[kVG][4];
#pragma unroll
                for (int j = 0; j < kVG; ++j) m3_ld4(xs + (int64_t)(l0 + min(r0 + j * vdr, nt - 1)) * p.proj_sl, x[j]);
#pragma unroll
                for (int j = 0; j < kVG; ++j) {
                    const int r = r0 + j * vdr;
                    if (r < nt) {
                        x[j][0] *= vmx.x; x[j][1] *= vmx.y; x[j][2] *= vmx.z; x[j][3] *= vmx.w;
                        m3_st4(static_cast<TO*>(p.v) + ((((int64_t)b * p.L + l0 + r) * M + vm) * p.H + h) * P + 4 * vpq,
                               x[j]);
                    }
                }
            }
        } else {
            for (int i = t; i < nt * M * PQ; i += 256) {
                const int pq = i % PQ, m = (i / PQ) % M, r = i / (PQ * M);
                float x[4];
                m3_ld4(projb + (int64_t)(l0 + r) * p.proj_sl + d_inner + h * P + 4 * pq, x);
                if (p.mx) {
                    const float4 mv = *(const float4*)(p.mx + ((int64_t)h * M + m) * P + 4 * pq);
                    x[0] *= mv.x; x[1] *= mv.y; x[2] *= mv.z; x[3] *= mv.w;
                }
                m3_st4(static_cast<TO*>(p.v) + ((((int64_t)b * p.L + l0 + r) * M + m) * p.H + h) * P + 4 * pq, x);
            }
        }
        if (t < nt) {
            const int64_t o = ((int64_t)b * p.L + l0 + t) * p.H + h;
            const float gmv = s_lam[t] * s_dt[t];
            p.da[o] = s_da[t];
            p.gm[o] = gmv;
            p.sc[o] = __builtin_fmaf(1.f - s_lam[t + 1], s_dt[t + 1], gmv);
        }
        // the rest of the cache tail: the last x and the wrapped angle
        if (l0 + nt == p.L) {
            for (int pp = t; pp < P; pp += 256)
                p.vst[bh * P + pp] = m3_ld1(projb + (int64_t)(p.L - 1) * p.proj_sl + d_inner + h * P + pp);
            if (t < A) p.ang_out[bh * A + t] = m3_ang_rad(theta);
        }
        __syncthreads();  // LDS reuse by the next tile
    }
}

// ---- epilogue ------------------------------------------------------------
struct M3FinishParams {
    int nb, L, H, P, M, YM;  // YM: ranks in y's rank axis (the first M are read)
    bool io_bf16, z_bf16, out_bf16;
    const void* y; const void* v;
    const void* z; int64_t z_sb, z_sl;
    const float* Dh; const float* mz; const float* mo; const float* onw;
    void* out; int64_t out_sb, out_sl;
};

__device__ __forceinline__ float m3f_ld(bool bf, const void* base, int64_t i) {
    return bf ? bf16_to_f32(static_cast<const bf16_t*>(base)[i]) : static_cast<const float*>(base)[i];
}

// ---- double-SSD pathway inputs -------------------------------------------
// One wave per (b, t, h): ranks m < M of the 2M-rank call carry gamma_t v_t
// with B_t, ranks M + m carry beta_t v_{t-1} with B_{t-1} (the cache's x_prev
// mimo_x and K_prev at t = 0); both carry C_t.  gamma = lambda dt and
// beta = (1 - lambda) dt exp(da) (trapezoidal_coefficients, helpers.rs:42-73).
struct M3DoubleParams {
    const void* v; const void* B; const void* C;
    const float* xp; const float* kp; const float* mx;
    void* v2; void* B2; void* C2;
};

__global__ __launch_bounds__(256) void mamba3_double_inputs_kernel(M3PrepParams p, M3DoubleParams d) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= (int64_t)p.nb * p.L * p.H) return;  // whole waves exit together
    const int h = (int)(item % p.H);
    const int64_t bl = item / p.H;
    const int t = (int)(bl % p.L), b = (int)(bl / p.L);
    const int M = p.M, H = p.H, P = p.P, N = p.N;
    float dt, da, lam;
    m3p_coef(p, b, t, h, dt, da, lam);
    const float gamma = lam * dt, beta = (1.f - lam) * dt * __expf(da);
    for (int m = 0; m < M; ++m) {
        const int64_t cur = ((bl * M + m) * H + h), prv = (((bl - 1) * M + m) * H + h);
        const int64_t o0 = ((bl * 2 * M + m) * H + h), o1 = ((bl * 2 * M + M + m) * H + h);
        for (int pp = lane; pp < P; pp += 64) {
            const float vt = m3f_ld(p.io_bf16, d.v, cur * P + pp);
            const float vp = t > 0 ? m3f_ld(p.io_bf16, d.v, prv * P + pp)
                                   : d.xp[((int64_t)b * H + h) * P + pp] * (d.mx ? d.mx[((int64_t)h * M + m) * P + pp] : 1.f);
            m3p_st(p.io_bf16, d.v2, o0 * P + pp, gamma * vt);
            m3p_st(p.io_bf16, d.v2, o1 * P + pp, beta * vp);
        }
        for (int n = lane; n < N; n += 64) {
            const float bt = m3f_ld(p.io_bf16, d.B, cur * N + n);
            const float bp = t > 0 ? m3f_ld(p.io_bf16, d.B, prv * N + n) : d.kp[(((int64_t)b * M + m) * H + h) * N + n];
            const float ct = m3f_ld(p.io_bf16, d.C, cur * N + n);
            m3p_st(p.io_bf16, d.B2, o0 * N + n, bt);
            m3p_st(p.io_bf16, d.B2, o1 * N + n, bp);
            m3p_st(p.io_bf16, d.C2, o0 * N + n, ct);
            m3p_st(p.io_bf16, d.C2, o1 * N + n, ct);
        }
    }
}

// one wave per (b, l, h); lanes over headdim (P <= 256, up to 4 per lane)
__global__ __launch_bounds__(256) void mamba3_finish_kernel(M3FinishParams p) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= (int64_t)p.nb * p.L * p.H) return;  // whole waves exit together
    const int h = (int)(item % p.H);
    const int64_t bl = item / p.H;
    const int l = (int)(bl % p.L), b = (int)(bl / p.L);
    const float Dv = p.Dh ? p.Dh[h] : 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int m = 0; m < p.M; ++m) {
        float o[4];
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int pp = lane + 64 * k;
            o[k] = 0.f;
            if (pp < p.P) {
                const int64_t yi = (((bl * p.YM + m) * p.H + h) * p.P) + pp;
                const int64_t vi = (((bl * p.M + m) * p.H + h) * p.P) + pp;
                o[k] = m3f_ld(p.io_bf16, p.y, yi);
                if (p.v) o[k] += Dv * m3f_ld(p.io_bf16, p.v, vi);
                ss += o[k] * o[k];
            }
        }
        float inv = 1.f;
        if (p.onw) inv = 1.f / sqrtf(wave_sum(ss) / (float)p.P + 8.1584695e-8f);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int pp = lane + 64 * k;
            if (pp >= p.P) continue;
            float zv = m3f_ld(p.z_bf16, p.z, (int64_t)b * p.z_sb + (int64_t)l * p.z_sl + h * p.P + pp);
            if (p.M > 1) zv *= p.mz[((int64_t)h * p.M + m) * p.P + pp];
            const float sz = zv / (1.f + __expf(-zv));
            float gv = p.onw ? (o[k] * inv) * p.onw[pp] * sz : o[k] * sz;
            if (p.M > 1) gv *= p.mo[((int64_t)h * p.M + m) * p.P + pp];
            acc[k] += gv;
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int pp = lane + 64 * k;
        if (pp < p.P)
            m3p_st(p.out_bf16, p.out, (int64_t)b * p.out_sb + (int64_t)l * p.out_sl + h * p.P + pp, acc[k]);
    }
}

constexpr int kM3PrepTS = 32;

int m3_prep_params(const mamba3_prep_args* a, M3PrepParams* out, bool need_outputs) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->nheads > 0 && a->headdim > 0 && a->ngroups > 0,
                    "sizes must be >= 1");
    MAMBA_CHECK_ARG(a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    MAMBA_CHECK_ARG(a->dstate == 8 || a->dstate == 16 || a->dstate == 32 || a->dstate == 64 || a->dstate == 128 ||
                        a->dstate == 256,
                    "dstate must be one of 8, 16, 32, 64, 128, 256");
    MAMBA_CHECK_ARG(a->headdim <= 1024, "headdim <= 1024 required");
    MAMBA_CHECK_ARG(a->mimo >= 1 && a->mimo <= 16, "mimo must be in [1, 16]");
    MAMBA_CHECK_ARG(a->rope_dim >= 0 && a->rope_dim <= a->dstate && a->rope_dim % 2 == 0,
                    "rope_dim must be even and in [0, dstate]");
    MAMBA_CHECK_ARG(a->angle_out && a->angle_out != a->angle, "angle_out is required and must not alias angle");
    MAMBA_CHECK_ARG(a->proj && a->ssm_state && a->k_state && a->v_state && a->angle && a->dt_bias &&
                        a->b_norm_w && a->c_norm_w && a->b_bias && a->c_bias && a->initial_state,
                    "proj, cache, parameters and initial_state are required");
    MAMBA_CHECK_ARG(!need_outputs || (a->v && a->B && a->C && a->da && a->gamma && a->scale),
                    "v, B, C, da, gamma and scale are required");
    MAMBA_CHECK_ARG(a->mimo == 1 || a->mimo_x, "mimo_x is required when mimo > 1");
    MAMBA_CHECK_ARG(a->proj_dtype == MAMBA_F32 || a->proj_dtype == MAMBA_BF16, "bad proj_dtype");
    MAMBA_CHECK_ARG(a->io_dtype == MAMBA_F32 || a->io_dtype == MAMBA_BF16, "bad io_dtype");
    M3PrepParams& p = *out;
    p.nb = a->batch; p.L = a->seqlen; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups; p.N = a->dstate;
    p.M = a->mimo; p.R = a->rope_dim; p.A = a->rope_dim / 2 > 1 ? a->rope_dim / 2 : 1;
    MAMBA_CHECK_ARG(p.A <= 256, "too many angles");
    const int64_t row = 2LL * p.H * p.P + 2LL * p.M * p.G * p.N + 3LL * p.H + p.A;
    MAMBA_CHECK_ARG(a->proj_sl >= row && (a->seqlen == 1 || a->proj_sb >= a->proj_sl), "proj strides too small");
    p.proj_bf16 = a->proj_dtype == MAMBA_BF16; p.io_bf16 = a->io_dtype == MAMBA_BF16;
    p.proj = a->proj; p.proj_sb = a->proj_sb; p.proj_sl = a->proj_sl;
    p.ssm = a->ssm_state; p.kst = a->k_state; p.vst = a->v_state; p.ang = a->angle; p.ang_out = a->angle_out;
    p.dt_bias = a->dt_bias; p.a_floor = a->a_floor; p.dt_lo = a->dt_min; p.dt_hi = a->dt_max;
    p.span = (float)((double)a->rotation_range * 3.14159265358979323846);
    p.bnw = a->b_norm_w; p.cnw = a->c_norm_w; p.bbias = a->b_bias; p.cbias = a->c_bias; p.mx = a->mimo_x;
    p.v = a->v; p.Bo = a->B; p.Co = a->C; p.da = a->da; p.gm = a->gamma; p.sc = a->scale; p.h0 = a->initial_state;
    return MAMBA_OK;
}

}  // namespace mamba

using namespace mamba;

// The fast path needs 16-byte aligned vector access to proj rows (B/C and x
// slices) and 4-wide headdim.
void mamba::m3_launch_seed(const M3PrepParams& p, hipStream_t s) {
    // rows per workgroup: at most kSeedE state elements per thread, at most P rows
    // (LDS <= M (P + N) floats, 32 KB at the limits M = 16, P = N = 256)
    int rows_per = (256 * kSeedE) / p.N > 0 ? (256 * kSeedE) / p.N : 1;
    rows_per = rows_per < p.P ? rows_per : p.P;
    hipLaunchKernelGGL(mamba3_seed_kernel, dim3(p.nb * p.H, (p.P + rows_per - 1) / rows_per), dim3(256),
                       (size_t)p.M * (rows_per + p.N) * sizeof(float), s, p, rows_per);
}

static bool m3_prep_fast(const M3PrepParams& p) {
    if (((uintptr_t)p.proj & 15u) != 0) return false;
    if (p.proj_sl % 8 != 0 || (p.nb > 1 && p.proj_sb % 8 != 0)) return false;
    if ((2 * p.H * p.P) % 8 != 0 || p.P % 4 != 0 || (p.H * p.P) % 4 != 0) return false;
    if (p.mx && ((uintptr_t)p.mx & 15u) != 0) return false;
    if (((uintptr_t)p.bbias & 15u) != 0 || ((uintptr_t)p.cbias & 15u) != 0) return false;
    if (((uintptr_t)p.kst & 15u) != 0) return false;
    if (((uintptr_t)p.v & 15u) != 0 || ((uintptr_t)p.Bo & 15u) != 0 || ((uintptr_t)p.Co & 15u) != 0) return false;
    // dynamic LDS of both kernels within 64 KB
    if ((size_t)kM3Tile * (((p.A + 3) & ~3) + p.N) * sizeof(float) > 64 * 1024) return false;
    if ((size_t)kM3Tile * (p.H + p.A) * sizeof(float) > 64 * 1024) return false;
    return true;
}
static int m3_seg_len(const M3PrepParams& p) {
    int seg = kM3Seg;
    while (seg > kM3Tile && (int64_t)p.nb * p.H * ((p.L + seg - 1) / seg) < 512) seg /= 2;
    return seg;
}
static int m3_nseg(const M3PrepParams& p) { return (p.L + m3_seg_len(p) - 1) / m3_seg_len(p); }

extern "C" int mamba3_prep_fast_path(const mamba3_prep_args* a) {
    M3PrepParams p;
    if (m3_prep_params(a, &p, true) != MAMBA_OK) return -1;
    return m3_prep_fast(p) ? 1 : 0;
}

extern "C" size_t mamba3_prep_workspace_size(const mamba3_prep_args* a) {
    M3PrepParams p;
    if (m3_prep_params(a, &p, true) != MAMBA_OK) return 0;
    const int nseg = m3_nseg(p);
    if (!m3_prep_fast(p) || nseg == 1) return 0;
    return (size_t)p.nb * nseg * p.H * p.A * sizeof(int);
}

template <typename TP, typename TO>
static void m3_launch_fast(const M3PrepParams& p, int* tot, hipStream_t s) {
    const int nseg = m3_nseg(p);
    if (nseg > 1) {
        const int hpw = p.A >= 256 ? 1 : (256 / p.A < p.H ? 256 / p.A : p.H);  // heads per workgroup
        hipLaunchKernelGGL((mamba3_angle_tot_kernel<TP>), dim3(p.nb * nseg, (p.H + hpw - 1) / hpw), dim3(256),
                           (size_t)kM3Tile * (hpw + p.A) * sizeof(float), s, p, nseg, m3_seg_len(p), hpw, tot);
    }
    const dim3 grid(p.nb * p.H * nseg), block(256);
    const size_t lds = (size_t)kM3Tile * (((p.A + 3) & ~3) + p.N) * sizeof(float);
#define MAMBA3_SEG_N(NN) \
    hipLaunchKernelGGL((mamba3_prep_seg_kernel<TP, TO, NN>), grid, block, lds, s, p, nseg, m3_seg_len(p), \
                       (const int*)tot);
    switch (p.N) {
        case 8: MAMBA3_SEG_N(8) break;
        case 16: MAMBA3_SEG_N(16) break;
        case 32: MAMBA3_SEG_N(32) break;
        case 64: MAMBA3_SEG_N(64) break;
        case 128: MAMBA3_SEG_N(128) break;
        default: MAMBA3_SEG_N(256) break;
    }
#undef MAMBA3_SEG_N
}

extern "C" int mamba3_prep_fwd(const mamba3_prep_args* a, void* workspace, size_t workspace_bytes,
                               mamba_stream_t stream) {
    M3PrepParams p;
    const int st = m3_prep_params(a, &p, true);
    if (st != MAMBA_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    const size_t need = mamba3_prep_workspace_size(a);
    MAMBA_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                    "workspace too small: mamba3_prep_workspace_size() bytes are required");
    MAMBA_CHECK_ARG(need == 0 || ((uintptr_t)workspace & 7u) == 0, "workspace must be 8-byte aligned");
    MAMBA_CHECK_ARG((int64_t)p.nb * p.H * m3_nseg(p) < (1ll << 31), "too many (batch, head, segment) items");
    m3_launch_seed(p, s);
    MAMBA_CHECK_LAUNCH();
    if (m3_prep_fast(p)) {
        int* tot = (int*)workspace;
        if (p.proj_bf16 && p.io_bf16) m3_launch_fast<bf16_t, bf16_t>(p, tot, s);
        else if (p.proj_bf16) m3_launch_fast<bf16_t, float>(p, tot, s);
        else if (p.io_bf16) m3_launch_fast<float, bf16_t>(p, tot, s);
        else m3_launch_fast<float, float>(p, tot, s);
        MAMBA_CHECK_LAUNCH();
        return MAMBA_OK;
    }
    const int npair = p.R / 2;
    auto lds_of = [&](int ts) {
        return (size_t)(2 * ts * p.N + 2 * ts * npair + ts * p.A + ts * p.P) * sizeof(float);
    };
    // wide tiles while the dynamic LDS stays within 64 KB
    const bool wide = lds_of(kM3PrepTS) <= 64 * 1024;
    const dim3 grid(p.nb * p.H * p.M), block(256);
#define MAMBA3_PREP_N(NN)                                                                                        \
    if (wide)                                                                                                    \
        hipLaunchKernelGGL((mamba3_prep_kernel<kM3PrepTS, NN>), grid, block, lds_of(kM3PrepTS), s, p);          \
    else                                                                                                         \
        hipLaunchKernelGGL((mamba3_prep_kernel<8, NN>), grid, block, lds_of(8), s, p);
    switch (p.N) {
        case 8: MAMBA3_PREP_N(8) break;
        case 16: MAMBA3_PREP_N(16) break;
        case 32: MAMBA3_PREP_N(32) break;
        case 64: MAMBA3_PREP_N(64) break;
        case 128: MAMBA3_PREP_N(128) break;
        default: MAMBA3_PREP_N(256) break;
    }
#undef MAMBA3_PREP_N
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

extern "C" int mamba3_finish_fwd(const mamba3_finish_args* a, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->nheads > 0 && a->headdim > 0 && a->headdim <= 256,
                    "sizes must be >= 1 and headdim <= 256");
    MAMBA_CHECK_ARG(a->mimo >= 1 && a->mimo <= 16, "mimo must be in [1, 16]");
    MAMBA_CHECK_ARG(a->mimo == 1 || (a->mimo_z && a->mimo_o), "mimo_z and mimo_o are required when mimo > 1");
    MAMBA_CHECK_ARG(a->y_ssd && a->z && a->out, "y_ssd, z and out are required");
    MAMBA_CHECK_ARG(a->v || !a->D, "v is required when D is given");
    MAMBA_CHECK_ARG((a->io_dtype == MAMBA_F32 || a->io_dtype == MAMBA_BF16) &&
                        (a->z_dtype == MAMBA_F32 || a->z_dtype == MAMBA_BF16) &&
                        (a->out_dtype == MAMBA_F32 || a->out_dtype == MAMBA_BF16),
                    "bad dtype");
    MAMBA_CHECK_ARG(a->y_ranks == 0 || (a->y_ranks >= a->mimo && a->y_ranks <= 32),
                    "y_ranks must be 0 or in [mimo, 32]");
    M3FinishParams p;
    p.nb = a->batch; p.L = a->seqlen; p.H = a->nheads; p.P = a->headdim; p.M = a->mimo;
    p.YM = a->y_ranks > 0 ? a->y_ranks : a->mimo;
    p.io_bf16 = a->io_dtype == MAMBA_BF16; p.z_bf16 = a->z_dtype == MAMBA_BF16; p.out_bf16 = a->out_dtype == MAMBA_BF16;
    p.y = a->y_ssd; p.v = a->v; p.z = a->z; p.z_sb = a->z_sb; p.z_sl = a->z_sl;
    p.Dh = a->D; p.mz = a->mimo_z; p.mo = a->mimo_o; p.onw = a->out_norm_w;
    p.out = a->out; p.out_sb = a->out_sb; p.out_sl = a->out_sl;
    const int64_t items = (int64_t)p.nb * p.L * p.H;
    MAMBA_CHECK_ARG((items + 3) / 4 < (1ll << 31), "too many (batch, position, head) items");
    hipLaunchKernelGGL(mamba3_finish_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, (hipStream_t)stream, p);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}

extern "C" int mamba3_double_inputs(const mamba3_double_inputs_args* a, mamba_stream_t stream) {
    MAMBA_CHECK_ARG(a != nullptr, "args is NULL");
    MAMBA_CHECK_ARG(a->batch > 0 && a->seqlen > 0 && a->nheads > 0 && a->headdim > 0 && a->dstate > 0,
                    "sizes must be >= 1");
    MAMBA_CHECK_ARG(a->ngroups > 0 && a->nheads % a->ngroups == 0, "nheads must be a multiple of ngroups");
    MAMBA_CHECK_ARG(a->mimo >= 1 && a->mimo <= 16, "mimo must be in [1, 16]");
    MAMBA_CHECK_ARG(a->mimo == 1 || a->mimo_x, "mimo_x is required when mimo > 1");
    MAMBA_CHECK_ARG(a->proj && a->dt_bias && a->v && a->B && a->C && a->x_prev && a->k_prev && a->v2 && a->B2 && a->C2,
                    "proj, dt_bias, v, B, C, x_prev, k_prev, v2, B2 and C2 are required");
    MAMBA_CHECK_ARG((a->proj_dtype == MAMBA_F32 || a->proj_dtype == MAMBA_BF16) &&
                        (a->io_dtype == MAMBA_F32 || a->io_dtype == MAMBA_BF16),
                    "bad dtype");
    M3PrepParams p{};
    p.nb = a->batch; p.L = a->seqlen; p.H = a->nheads; p.P = a->headdim; p.G = a->ngroups; p.N = a->dstate;
    p.M = a->mimo;
    p.proj_bf16 = a->proj_dtype == MAMBA_BF16; p.io_bf16 = a->io_dtype == MAMBA_BF16;
    p.proj = a->proj; p.proj_sb = a->proj_sb; p.proj_sl = a->proj_sl;
    p.dt_bias = a->dt_bias; p.a_floor = a->a_floor; p.dt_lo = a->dt_min; p.dt_hi = a->dt_max;
    M3DoubleParams d;
    d.v = a->v; d.B = a->B; d.C = a->C; d.xp = a->x_prev; d.kp = a->k_prev; d.mx = a->mimo_x;
    d.v2 = a->v2; d.B2 = a->B2; d.C2 = a->C2;
    const int64_t items = (int64_t)p.nb * p.L * p.H;
    MAMBA_CHECK_ARG((items + 3) / 4 < (1ll << 31), "too many (batch, position, head) items");
    hipLaunchKernelGGL(mamba3_double_inputs_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, p, d);
    MAMBA_CHECK_LAUNCH();
    return MAMBA_OK;
}
