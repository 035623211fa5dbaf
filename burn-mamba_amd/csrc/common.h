// Shared host/device helpers for the gfx950 SSM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "../../include/mamba_hip.h"

namespace mamba {

// ---------------------------------------------------------------- errors ---
void set_error(const std::string& msg);

#define MAMBA_CHECK_ARG(cond, msg)                                  \
    do {                                                            \
        if (!(cond)) {                                              \
            ::mamba::set_error(std::string(__func__) + ": " + msg); \
            return MAMBA_ERR_INVALID_ARG;                           \
        }                                                           \
    } while (0)

#define MAMBA_CHECK_HIP(expr)                                                         \
    do {                                                                              \
        hipError_t e_ = (expr);                                                       \
        if (e_ != hipSuccess) {                                                       \
            ::mamba::set_error(std::string(__func__) + ": " #expr " -> " +          \
                               hipGetErrorString(e_));                                \
            return MAMBA_ERR_HIP;                                                     \
        }                                                                             \
    } while (0)

#define MAMBA_CHECK_LAUNCH() MAMBA_CHECK_HIP(hipGetLastError())

// ----------------------------------------------------------------- bf16 ---
typedef uint16_t bf16_t;  // storage type; arithmetic always in f32

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
    return __uint_as_float(((uint32_t)v) << 16);
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    // round to nearest even; NaN stays NaN (quiet bit kept by the high half)
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (bf16_t)(u >> 16);
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_f32<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__device__ __forceinline__ void store_f32(T* p, float v);
template <>
__device__ __forceinline__ void store_f32<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_f32<bf16_t>(bf16_t* p, float v) { *p = f32_to_bf16(v); }

// ------------------------------------------------------------ numerics ---
// softplus with the f32 threshold of src/modules/activation/softplus.rs:21-47
__device__ __forceinline__ float softplus_f32(float x) {
    const float thr = 18.f;
    return x > thr ? x : log1pf(expf(fminf(x, thr)));
}
// silu(x) = x / (1 + exp(-x))  (src/modules/activation/silu.rs:24-27)
__device__ __forceinline__ float silu_f32(float x) { return x / (expf(-x) + 1.f); }
// div_eps(F32) of src/utils/mod.rs:59-65
constexpr float kDivEpsF32 = 8.1584695e-8f;

// The generic SSD chunk-state kernels take wide slices (32 entries per thread)
// when (head, chunk, batch) alone gives at least this many workgroups.
constexpr int64_t kGenericStateWide = 2048;

// ---------------------------------------------------- wave/block scans ---
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Inclusive prefix sum over a wave (64 lanes), on DPP lane moves (no LDS
// round trips): shifts by 1, 2, 4, 8 inside each 16-lane row, then lane 15 of
// each row broadcast into the next row and lane 31 into the upper half.
// Lanes with no source add 0 (bound_ctrl / masked rows keep the old value 0).
__device__ __forceinline__ float dpp_term(float v, int ctrl, int row_mask) {
    switch (ctrl) {  // the DPP control is an immediate
        case 0x111: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false));
        case 0x112: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, false));
        case 0x114: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, false));
        case 0x118: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, false));
        case 0x142: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
        default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));
    }
}
// Sum over aligned groups of G lanes (G a power of two, <= 64) into each
// group's last lane, on the same DPP moves: after the row shifts by 1 .. G/2
// lane i holds the sum of lanes i - G + 1 .. i of its row, which for the last
// lane of a group is the group; groups of 32 and 64 add the row broadcasts.
// The other lanes hold partial sums.  (A __shfl_xor butterfly gives every
// lane the sum but costs one LDS permute per step.)
template <int G>
__device__ __forceinline__ float group_sum_last(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "group size must be a power of two <= 64");
    if (G >= 2) v += dpp_term(v, 0x111, 0xf);   // row_shr:1
    if (G >= 4) v += dpp_term(v, 0x112, 0xf);   // row_shr:2
    if (G >= 8) v += dpp_term(v, 0x114, 0xf);   // row_shr:4
    if (G >= 16) v += dpp_term(v, 0x118, 0xf);  // row_shr:8
    if (G >= 32) v += dpp_term(v, 0x142, 0xa);  // row_bcast:15 into rows 1 and 3
    if (G >= 64) v += dpp_term(v, 0x143, 0xc);  // row_bcast:31 into rows 2 and 3
    return v;
}
// Wave sum as a wave-uniform value: the DPP group sum into lane 63, read
// back as a scalar.  Every lane of the wave must be active.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_sum_last<64>(v)), 63));
}
// Inclusive prefix sum over the wave.  The input is made opaque first: a
// caller's product (a scan of dt A) would otherwise be contracted into the
// first add as an fma in some kernels and not in others, and kernels that
// must agree bit for bit scan the same values.
__device__ __forceinline__ float wave_incl_scan(float v) {
    asm volatile("" : "+v"(v));
    v += dpp_term(v, 0x111, 0xf);  // row_shr:1
    v += dpp_term(v, 0x112, 0xf);  // row_shr:2
    v += dpp_term(v, 0x114, 0xf);  // row_shr:4
    v += dpp_term(v, 0x118, 0xf);  // row_shr:8
    v += dpp_term(v, 0x142, 0xa);  // row_bcast:15 into rows 1 and 3
    v += dpp_term(v, 0x143, 0xc);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Wave index inside the workgroup, as a wave-uniform (scalar) value: branches
// and loops on it stay scalar, so waits on memory counters remain exact.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// --------------------------------------------------- streamed state tiles ---
// 16-byte loads and stores with the non-temporal hint, for data touched once
// per launch (a decode state tile read and written back): it then does not
// displace the caches' reusable lines (weights, partial planes, activations).
typedef float nt_f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt4(const float4* p) {
    const nt_f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4_t*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt4(float4* p, float4 h) {
    const nt_f32x4_t v = {h.x, h.y, h.z, h.w};
    __builtin_nontemporal_store(v, reinterpret_cast<nt_f32x4_t*>(p));
}

// ------------------------------------------------------- buffer access ---
// Raw buffer resources (gfx9 descriptor word 3): loads at or past `bytes` read
// as zero and stores there are dropped, which clips tiles at a sequence end
// without per-lane bounds checks.  `base` and `bytes` must be wave-uniform:
// they are read from the first active lane, so the descriptor is scalar.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    void* ub = (void*)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// per-lane offset `off` plus a wave-uniform offset `soff` (a scalar operand)
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                         r, off, (int)__builtin_amdgcn_readfirstlane(soff), 0));
}
// the same with the non-temporal hint (data streamed once)
__device__ __forceinline__ uint4 buf_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                         r, off, (int)__builtin_amdgcn_readfirstlane(soff), 2));
}
__device__ __forceinline__ float buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint2 buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint16_t buf_ld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
__device__ __forceinline__ void buf_st8(__amdgpu_buffer_rsrc_t r, uint32_t off, uint2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(
        __builtin_bit_cast(decltype(__builtin_amdgcn_raw_buffer_load_b64(r, 0, 0, 0)), v), r, off, 0, 0);
}

// Raw buffer resource words (base, num_records, the flags buf_rsrc uses), in
// scalar registers: `base` and `bytes` must be wave-uniform.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4_t buf_words(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    u32x4_t w;
    w.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
    w.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu;  // stride 0
    w.z = __builtin_amdgcn_readfirstlane(bytes);
    w.w = 0x00020000u;
    return w;
}

// One direct-to-LDS load of 16 bytes per lane: bytes [soff + voff, +16) of
// the buffer (zero past its end) land at LDS address lds + 16 * lane.  `lds`
// and `soff` are wave-uniform.  Written as inline assembly so that the
// compiler's memory-counter bookkeeping does not see it: its own LDS
// accesses are then never held back by these loads (it cannot always prove
// them disjoint), and the caller waits for them (an s_waitcnt on the vector
// memory counter that covers them, then a barrier) before anything reads the
// destination.  The compiler's own vmcnt waits stay correct: the counter
// drains in issue order, so an uncounted load can only make them wait longer.
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, %3 offen lds"
        :
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(rsrc), "s"(soff)
        : "m0");
}

// two floats -> two bf16 (round to nearest even) in one dword, lo first
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace mamba
