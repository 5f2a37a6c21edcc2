// Device helpers shared by the QORA decode kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "params.hpp"

namespace qora {

constexpr int kWave = 64;

// IEEE binary16 -> binary32 (exact; v_cvt_f32_f16).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// binary32 -> binary16, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f2h(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// ---- Q4 nibbles as exact binary16 values ----
// A 32-bit word of packed weights holds 8 columns: byte i carries column 2i
// in its low nibble and column 2i+1 in its high nibble. OR-ing a nibble
// into the mantissa of a binary16 with a fixed exponent gives an exact small
// integer: 0x6400 | q = 1024 + q and 0x5400 | (q << 4) = 64 + q, and one
// v_pk_add_f16 takes the bias off both halves exactly (q - 8 is an integer
// in [-8, 7]). One v_and_or_b32 builds two values (one per 16-bit half), and
// v_fma_mix_f32 multiplies a half by an fp32 operand into an fp32
// accumulator, so each product is the exact (q - 8) * x of the reference
// arithmetic: 17 VALU instructions per 8 nibbles instead of 24 (extract,
// convert, multiply-add).
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

struct NibbleConsts {
    uint32_t m_lo, m_hi;   // nibble masks (scalar registers)
    uint32_t e_lo, e_hi;   // binary16 exponent patterns (vector registers)
};

__device__ __forceinline__ NibbleConsts nibble_consts() {
    NibbleConsts k{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
    // Register operands let the backend select a single v_and_or_b32 (gfx9
    // VOP3 instructions take no literal constants).
    asm volatile("" : "+s"(k.m_lo), "+s"(k.m_hi));
    asm volatile("" : "+v"(k.e_lo), "+v"(k.e_hi));
    return k;
}

struct Nib8 {
    uint32_t c04, c15, c26, c37;   // binary16 pairs: (column a | column b << 16)
};

template <int BIAS>
__device__ __forceinline__ uint32_t f16x2_minus(uint32_t v) {
    half2v h = __builtin_bit_cast(half2v, v);
    h = h - (half2v){(_Float16)(float)BIAS, (_Float16)(float)BIAS};
    return __builtin_bit_cast(uint32_t, h);
}

// Columns (0|4), (1|5), (2|6), (3|7) of the word as binary16 pairs of q - 8.
__device__ __forceinline__ Nib8 unpack_nibbles(uint32_t w, const NibbleConsts& k) {
    const uint32_t s = w >> 8;
    Nib8 n;
    n.c04 = f16x2_minus<1032>((w & k.m_lo) | k.e_lo);
    n.c15 = f16x2_minus<72>((w & k.m_hi) | k.e_hi);
    n.c26 = f16x2_minus<1032>((s & k.m_lo) | k.e_lo);
    n.c37 = f16x2_minus<72>((s & k.m_hi) | k.e_hi);
    return n;
}

__device__ __forceinline__ float f16lo(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
}

__device__ __forceinline__ float f16hi(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}


// Fixed-point accumulator values (params.hpp): int64 / 2^36.
__device__ __forceinline__ long long to_fixed(float v) {
    return __double2ll_rn((double)v * kFixScale);
}

// Kernel arguments are read by scalar loads that the compiler places next to
// each field's first use, each waited for on its own: a chain of memory round
// trips before a kernel's first large load (the argument lines do not stay
// cached across launches). kernarg_warm(p) reads one dword of every 64-byte
// line of the argument block in one statement, so all the line misses go out
// together and are waited for once; later field reads hit the scalar cache.
template <typename T>
__device__ __forceinline__ void kernarg_warm(const T& p) {
    static_assert(sizeof(T) % 4 == 0 && sizeof(T) <= 512, "argument block of at most 512 bytes");
    constexpr int N = (int)(sizeof(T) / 4);
    constexpr int I1 = 16 < N ? 16 : N - 1, I2 = 32 < N ? 32 : N - 1, I3 = 48 < N ? 48 : N - 1;
    constexpr int I4 = 64 < N ? 64 : N - 1, I5 = 80 < N ? 80 : N - 1, I6 = 96 < N ? 96 : N - 1;
    constexpr int I7 = 112 < N ? 112 : N - 1;
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&p);
    asm volatile("" ::"s"(w[0]), "s"(w[I1]), "s"(w[I2]), "s"(w[I3]), "s"(w[I4]), "s"(w[I5]), "s"(w[I6]), "s"(w[I7]),
                 "s"(w[N - 1]));
}

// Makes v a value the code below cannot re-load or move above this point:
// its load is issued and waited for here.
template <typename T>
__device__ __forceinline__ void sgpr_pin(T& v) {
    asm volatile("" : "+s"(v));
}

// A wave-uniform pointer held in scalar registers from here on: the asm
// keeps the compiler from re-reading it from the kernel arguments later.
// It must point to global memory (it is rebuilt as a global-address-space
// pointer, so accesses through it stay global instructions, not flat ones).
template <typename T>
__device__ __forceinline__ T* sgpr_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    asm volatile("" : "+s"(lo), "+s"(hi));
    using G = __attribute__((address_space(1))) T;
    G* g = (G*)(((uint64_t)hi << 32) | lo);
    return (T*)g;
}

// A wave-uniform int32 read with a scalar load (through the constant address
// space): its wait counts scalar loads only, so vector loads issued before it
// stay in flight while it is waited for. The value must not change while the
// kernel runs (the scalar cache is invalidated at each kernel start).
__device__ __forceinline__ int32_t ld_scalar_i32(const int32_t* p) {
    using C = const __attribute__((address_space(4))) int32_t;
    return *(C*)reinterpret_cast<uint64_t>(p);
}

__device__ __forceinline__ float from_fixed(long long a) {
    return (float)((double)a * (1.0 / kFixScale));
}

// Weight-stream loads, marked non-temporal: the weights of a decode step are
// read once per token, so they should not push the step's small, reused
// lines (kernel code, arguments, accumulators, KV rows) out of the L2.
typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));
typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_stream(const void* p) {
    const v4u32 v = __builtin_nontemporal_load(reinterpret_cast<const v4u32*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream2(const void* p) {
    const v2u32 v = __builtin_nontemporal_load(reinterpret_cast<const v2u32*>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_stream1(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// Range guard of the fixed-point accumulators (kFixReadLimit, kFixAddLimit).
__device__ __forceinline__ bool fix_out_of_range(long long a, long long lim) { return a >= lim || a <= -lim; }
__device__ __forceinline__ void fix_flag(int* flag, bool bad) {
    if (bad && flag) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-lane reductions over a wave64 with DPP (no LDS round trips): two
// quad permutes and two row rotates give every lane the total of its
// 16-lane row, then the four row totals are read with v_readlane and
// combined in a fixed order, so every lane receives the same value. Must be
// called with all 64 lanes active (wave-uniform control flow).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Positions per attention split at context length L: the smallest multiple of
// kAttnSub that keeps the number of splits within kAttnMaxSplits.
__host__ __device__ __forceinline__ uint32_t attn_chunk_for(uint32_t L) {
    const uint32_t c = (L + kAttnMaxSplits - 1) / kAttnMaxSplits;
    return c <= (uint32_t)kAttnSub ? (uint32_t)kAttnSub : (c + kAttnSub - 1) / kAttnSub * kAttnSub;
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);   // row_ror:4
    v += dpp_f32<0x128>(v);   // row_ror:8
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

// Sum over each 16-lane row by a DPP butterfly (no LDS): lane ^ 1, lane ^ 2,
// then the mirrored quad and the mirrored half row. Each step adds two
// equal-bit operands in either order, so all 16 lanes end with identical bits.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);   // row_half_mirror
    v += dpp_f32<0x140>(v);   // row_mirror
    return v;
}

// Sum of v over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four row slots of a
// wave), the same bits in all four: each lane-swap instruction leaves lane l's
// partner value in one of its two results, so their sum is v[l] + v[l ^ 16]
// (then ^ 32) in every lane.
__device__ __forceinline__ float sum_row_slots(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The same for the maximum.
__device__ __forceinline__ float max_row_slots(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Maximum over each aligned group of N lanes (N = 16: a row; 32: two rows),
// every lane of the group receiving it: the row16_sum butterfly with fmaxf,
// then the lane-swap of rows l and l ^ 16. All 64 lanes must be active.
template <int N>
__device__ __forceinline__ float group_max(float v) {
    static_assert(N == 16 || N == 32, "16- or 32-lane groups");
    v = fmaxf(v, dpp_f32<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140>(v));   // row_mirror
    if constexpr (N == 32) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x124>(v));
    v = fmaxf(v, dpp_f32<0x128>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

// RMSNorm factor 1 / sqrt(sum(x^2) / n + 1e-6) (rms_norm_f16, gemv.rs:744-753)
// from `parts` partial sums of squares (lane i loads partial i; parts <= 64).
__device__ __forceinline__ float rms_inv_from_parts(const float* ss, uint32_t parts, uint32_t n) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const float v = lane < parts ? ss[lane] : 0.f;
    const float total = wave_sum(v);
    return 1.0f / sqrtf(total / (float)n + 1e-6f);
}

// Block-wide sum for blockDim.x == NT (multiple of 64). `red` must hold
// NT/64 floats of shared memory. Every thread receives the total.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NT / kWave; ++i) t += red[i];
    return t;
}

// Candidate rule of the greedy sampler (generate.rs:346-352): a logit can
// win only if it is > -inf (so NaN and -inf never win); larger value wins,
// ties go to the lower index.
__device__ __forceinline__ bool argmax_better(float va, uint32_t ia, float vb, uint32_t ib) {
    const bool a_ok = va > -INFINITY;
    const bool b_ok = vb > -INFINITY;
    if (!a_ok) return false;
    if (!b_ok) return true;
    return va > vb || (va == vb && ia < ib);
}

}  // namespace qora
