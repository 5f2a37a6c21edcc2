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

// Byte B of a 32-bit word as float. The AMDGPU backend selects
// v_cvt_f32_ubyte{B} for this pattern (one instruction).
template <int B>
__device__ __forceinline__ float ubyte_f(uint32_t w) {
    return (float)((w >> (8 * B)) & 0xFFu);
}

// Fixed-point accumulator values (params.hpp): int64 / 2^36.
__device__ __forceinline__ long long to_fixed(float v) {
    return __double2ll_rn((double)v * kFixScale);
}

__device__ __forceinline__ float from_fixed(long long a) {
    return (float)((double)a * (1.0 / kFixScale));
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
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

// Device-scope release/acquire around the "last workgroup finishes the
// reduction" pattern. Workgroups of one launch run on different XCDs with
// separate L2s; the agent-scope fences write back / invalidate so the
// partials written by one XCD are visible to another.
__device__ __forceinline__ uint32_t arrive_counter(uint32_t* counter) {
    __threadfence();
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_u32_release(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qora
