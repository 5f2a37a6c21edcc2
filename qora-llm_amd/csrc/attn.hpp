// Decode-step kernels other than the GEMVs: GQA decode attention over the
// device KV cache, embedding row lookup, and standalone RMSNorm / RoPE /
// argmax used by the kernel-level entry points.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace qora {

// ---------------------------------------------------------------------------
// GQA decode attention (gemv.rs:914-989 + softmax_raw gemv.rs:782-793).
// Head h reads KV head h / groups. The KV cache is token-major
// [capacity][kv_heads][head_dim] (RawKvCache, gemv.rs:154-156), f32 or f16.
// Split-K over positions ("flash decoding"): block (s, kvh) takes CHUNK
// positions, stages K and V in LDS, computes the scores of all `groups`
// query heads of that KV head, and writes an unnormalised partial
// (max, sum of exp, sum of exp*V). The last block of a KV head merges the
// partials of the active splits in split order (deterministic).
// The length L = *pos + 1 is read on the device, so the launch shape is
// fixed for a given capacity and the step can be replayed from a graph.
// Limits (checked on the host): head_dim <= 128, groups <= 4, CHUNK = 32.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void attn_decode_kernel(AttnParams p) {
    constexpr int NT = 256;
    constexpr int C = kAttnChunk;
    constexpr int KS = kAttnMaxHd + 1;   // padded LDS row
    __shared__ float ks[C * KS];
    __shared__ float vs[C * kAttnMaxHd];
    __shared__ float qs[kAttnMaxGroups * kAttnMaxHd];
    __shared__ float sc[kAttnMaxGroups * C];
    __shared__ float smax[kAttnMaxGroups];
    __shared__ float ssum[kAttnMaxGroups];
    __shared__ int s_last;

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t L = p.pos ? (uint32_t)(*p.pos) + 1u : p.L;
    const uint32_t s_act = (L + C - 1) / C;
    if (split >= s_act) return;
    const uint32_t hd = p.hd, G = p.groups;
    const uint32_t p0 = split * C;
    const uint32_t cn = min((uint32_t)C, L - p0);
    const uint64_t kv_stride = (uint64_t)p.KVH * hd;

    // stage K, V rows [p0, p0+cn) of this KV head and the group's q heads
    for (uint32_t i = t; i < (uint32_t)C * hd; i += NT) {
        const uint32_t r = i / hd, d = i % hd;
        float kv = 0.f, vv = 0.f;
        if (r < cn) {
            const uint64_t idx = (uint64_t)(p0 + r) * kv_stride + (uint64_t)kvh * hd + d;
            if (p.kv_f16) {
                kv = h2f(reinterpret_cast<const uint16_t*>(p.kc)[idx]);
                vv = h2f(reinterpret_cast<const uint16_t*>(p.vc)[idx]);
            } else {
                kv = reinterpret_cast<const float*>(p.kc)[idx];
                vv = reinterpret_cast<const float*>(p.vc)[idx];
            }
        }
        ks[r * KS + d] = kv;
        vs[r * kAttnMaxHd + d] = vv;
    }
    for (uint32_t i = t; i < G * hd; i += NT) qs[i] = p.q[(uint64_t)(kvh * G) * hd + i];
    __syncthreads();

    // scores[g][r] = (q_g . k_r) * scale
    for (uint32_t i = t; i < G * C; i += NT) {
        const uint32_t g = i / C, r = i % C;
        float dot = 0.f;
        if (r < cn) {
            const float* kr = ks + r * KS;
            const float* qg = qs + g * hd;
            for (uint32_t d = 0; d < hd; ++d) dot = fmaf(qg[d], kr[d], dot);
            dot *= p.scale;
        }
        sc[g * C + r] = dot;
    }
    __syncthreads();
    // per head: max and sum of exp over the chunk (one wave per head)
    for (uint32_t g = wave; g < G; g += NT / kWave) {
        const float v = (lane < (int)cn) ? sc[g * C + lane] : -INFINITY;
        const float m = wave_max(v);
        const float e = (lane < (int)cn) ? expf(v - m) : 0.f;
        const float s = wave_sum(e);
        if (lane < C) sc[g * C + lane] = e;
        if (lane == 0) { smax[g] = m; ssum[g] = s; }
    }
    __syncthreads();
    // unnormalised output: sum_r e[g][r] * V[r][d]
    float* part = p.part + (((uint64_t)kvh * p.s_max + split) * G) * (hd + 2);
    for (uint32_t i = t; i < G * hd; i += NT) {
        const uint32_t g = i / hd, d = i % hd;
        float acc = 0.f;
        for (uint32_t r = 0; r < cn; ++r) acc = fmaf(sc[g * C + r], vs[r * kAttnMaxHd + d], acc);
        part[g * (hd + 2) + d] = acc;
    }
    if (t < (int)G) {
        part[t * (hd + 2) + hd] = smax[t];
        part[t * (hd + 2) + hd + 1] = ssum[t];
    }
    __threadfence();
    __syncthreads();
    if (t == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&p.counters[kvh], 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == s_act - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    // merge the s_act partials of every head of this KV head
    const float* base = p.part + ((uint64_t)kvh * p.s_max * G) * (hd + 2);
    for (uint32_t i = t; i < G * hd; i += NT) {
        const uint32_t g = i / hd, d = i % hd;
        float m = -INFINITY;
        for (uint32_t s = 0; s < s_act; ++s) m = fmaxf(m, base[(s * G + g) * (hd + 2) + hd]);
        float num = 0.f, den = 0.f;
        for (uint32_t s = 0; s < s_act; ++s) {
            const float* ps = base + (s * G + g) * (hd + 2);
            const float w = expf(ps[hd] - m);
            num = fmaf(ps[d], w, num);
            den = fmaf(ps[hd + 1], w, den);
        }
        p.out[(uint64_t)(kvh * G + g) * hd + d] = num / den;
    }
    if (t == 0) store_u32_release(&p.counters[kvh], 0u);
}

// ---------------------------------------------------------------------------
// Embedding row (embed_lookup, gemv.rs:515-526, 710-736): x = dequant(E[tok]).
// The token is read on the device: tok = src[idx ? *idx : 0].
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void embed_kernel(EmbedParams p) {
    int32_t tok = p.tok_src[p.tok_idx ? *p.tok_idx : 0];
    tok = tok < 0 ? 0 : (tok >= (int32_t)p.vocab ? (int32_t)p.vocab - 1 : tok);
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < p.hidden; j += gridDim.x * blockDim.x) {
        float v;
        if (p.fmt == 1) {
            const uint64_t G = p.hidden / 32;
            const uint8_t b = p.w[(uint64_t)tok * G * 16 + j / 2];
            const int q = (j & 1) ? (b >> 4) : (b & 0x0F);
            v = h2f(p.scales[(uint64_t)tok * G + j / 32]) * (float)(q - 8);
        } else {
            v = h2f(reinterpret_cast<const uint16_t*>(p.w)[(uint64_t)tok * p.hidden + j]);
        }
        p.x[j] = v;
    }
}

// Full-matrix Q4 dequant: out[i][j] = f32(scale[i][j/32]) * (q[i][j] - 8).
__global__ __launch_bounds__(256) void dequant_q4_kernel(const uint8_t* packed, const uint16_t* scales,
                                                         uint64_t k, uint64_t n, float* out) {
    const uint64_t total_bytes = k * n / 2;
    const uint64_t G = n / 32;
    for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total_bytes;
         b += (uint64_t)gridDim.x * blockDim.x) {
        const uint8_t v = packed[b];
        const uint64_t row = b / (n / 2);
        const uint64_t col = (b % (n / 2)) * 2;
        const float s = h2f(scales[row * G + col / 32]);
        out[row * n + col] = s * (float)((int)(v & 0x0F) - 8);
        out[row * n + col + 1] = s * (float)((int)(v >> 4) - 8);
    }
}

// Standalone RMSNorm (rms_norm_f16, gemv.rs:744-753), one block per vector.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* x, const uint16_t* gamma, uint32_t n,
                                                      float* out) {
    __shared__ float wred[4];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) { const float v = x[i]; ss += v * v; }
    ss = block_sum<256>(ss, wred);
    const float inv = 1.0f / sqrtf(ss / (float)n + 1e-6f);
    for (uint32_t i = threadIdx.x; i < n; i += 256) out[i] = x[i] * inv * h2f(gamma[i]);
}

// Standalone RoPE (apply_rope_raw, gemv.rs:757-778), in place.
__global__ __launch_bounds__(256) void rope_kernel(float* data, uint32_t num_heads, uint32_t head_dim,
                                                   const float* cos_t, const float* sin_t, uint32_t half,
                                                   uint32_t position) {
    const uint32_t total = num_heads * half;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const uint32_t h = i / half, d = i % half;
        float* b = data + (uint64_t)h * head_dim;
        const float x1 = b[d], x2 = b[half + d];
        const float c = cos_t[(uint64_t)position * half + d];
        const float s = sin_t[(uint64_t)position * half + d];
        b[d] = x1 * c - x2 * s;
        b[half + d] = x2 * c + x1 * s;
    }
}

// Standalone greedy argmax over a logits vector (generate.rs:346-352):
// one block, 256 threads.
__global__ __launch_bounds__(256) void argmax_kernel(const float* logits, uint32_t n, int32_t* out) {
    __shared__ float s_val[4];
    __shared__ uint32_t s_idx[4];
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
        const float v = logits[i];
        if (argmax_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const uint32_t oi = __shfl_xor(bi, off, kWave);
        if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x / 64;
    if (lane == 0) { s_val[wave] = bv; s_idx[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v0 = s_val[0];
        uint32_t i0 = s_idx[0];
        for (int w = 1; w < 4; ++w)
            if (argmax_better(s_val[w], s_idx[w], v0, i0)) { v0 = s_val[w]; i0 = s_idx[w]; }
        *out = (i0 == 0xFFFFFFFFu) ? 0 : (int32_t)i0;
    }
}

// End of a decode step that produced no logits (prefill positions):
// pos += 1. Single thread.
__global__ void advance_pos_kernel(int32_t* pos) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *pos = *pos + 1;
}

}  // namespace qora
