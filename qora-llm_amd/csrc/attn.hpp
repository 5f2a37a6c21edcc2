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
// Split over positions ("flash decoding"): block (s, kvh) takes `chunk`
// positions in sub-chunks of 32 staged in LDS, runs an online softmax for
// the `groups` query heads of that KV head and writes an unnormalised
// partial (running max m, sum of exp l, sum of exp*V). The partials are
// merged by the consumer (the o-projection prologue, or
// attn_combine_kernel for the kernel-level entry point), in split order.
// Model mode (qkv_acc set): q, k, v are read from the fixed-point q|k|v
// accumulator of the QKV GEMV; q and k are rotated (apply_rope_raw at the
// position being appended, gemv.rs:903-906) and the block that owns the new
// position writes its K and V rows into the cache (gemv.rs:909-911).
// L = *pos + 1 is read on the device, so the launch shape is fixed for a
// given capacity and the step can be replayed from a graph.
// Limits (checked on the host): head_dim <= 128, groups <= 4.
// ---------------------------------------------------------------------------

// Rotated value of dim d of a head whose un-rotated values are v[0..hd).
__device__ __forceinline__ float rope_at(const float* v, uint32_t d, uint32_t half, const float* ct,
                                         const float* st) {
    if (d < half) return v[d] * ct[d] - v[d + half] * st[d];
    if (d < 2 * half) return v[d] * ct[d - half] + v[d - half] * st[d - half];
    return v[d];
}

template <int DPL>
__device__ __forceinline__ void load_v_row(const AttnParams& p, uint64_t idx, float* v) {
    if (p.kv_f16) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(p.vc) + idx;
#pragma unroll
        for (int i = 0; i < DPL; ++i) v[i] = h2f(src[i]);
    } else {
        const float* src = reinterpret_cast<const float*>(p.vc) + idx;
        if constexpr (DPL == 2) {
            const float2 f = *reinterpret_cast<const float2*>(src);
            v[0] = f.x;
            v[1] = f.y;
        } else {
            v[0] = src[0];
        }
    }
}

// One wave per query head; lanes (half, r) = (lane / 32, lane % 32) own
// position c0 + r and half of the head dims for q.k, then lanes own DPL
// dims each for p.V. K and V are read straight from the cache (all loads of
// a 32-position pass are issued before the math). No block-wide barrier
// inside the position loop: each wave runs its own online softmax.
template <int DPL>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnParams p) {
    constexpr int NT = 256;
    constexpr int SUB = kAttnSub;                    // positions per pass (32)
    __shared__ float qs[kAttnMaxGroups * kAttnMaxHd];
    __shared__ float raw[(kAttnMaxGroups + 2) * kAttnMaxHd];
    __shared__ float knew[kAttnMaxHd];
    __shared__ float vnew[kAttnMaxHd];
    __shared__ float es[kAttnMaxGroups * SUB];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t L = p.pos ? (uint32_t)(*p.pos) + 1u : p.L;
    const uint32_t p0 = split * p.chunk;
    if (p0 >= L) return;
    const uint32_t p1 = min(L, p0 + p.chunk);
    const uint32_t hd = p.hd, G = p.groups;
    const uint64_t kv_stride = (uint64_t)p.KVH * hd;
    const uint32_t cur = L - 1;                        // position appended this step
    const bool model = p.qkv_acc != nullptr;
    const bool has_new = model && cur >= p0 && cur < p1;

    // ---- q of the group's heads (and the new k, v) ----
    if (model) {
        // the q|k|v GEMV ran on x * gamma; its RMSNorm factor is applied here
        const float inv = rms_inv_from_parts(p.ss_in, p.ss_n, p.norm_n);
        const uint32_t qd = p.H * hd;
        for (uint32_t i = t; i < G * hd; i += NT)
            raw[i] = inv * from_fixed(p.qkv_acc[(uint64_t)kvh * G * hd + i]);
        if (has_new)
            for (uint32_t d = t; d < hd; d += NT) {
                raw[G * hd + d] = inv * from_fixed(p.qkv_acc[qd + (uint64_t)kvh * hd + d]);
                raw[(G + 1) * hd + d] = inv * from_fixed(p.qkv_acc[qd + kv_stride + (uint64_t)kvh * hd + d]);
            }
        __syncthreads();
        const float* ct = p.rope_cos + (uint64_t)cur * p.half;
        const float* st = p.rope_sin + (uint64_t)cur * p.half;
        for (uint32_t i = t; i < G * hd; i += NT)
            qs[i] = p.use_rope ? rope_at(raw + (i / hd) * hd, i % hd, p.half, ct, st) : raw[i];
        if (has_new)
            for (uint32_t d = t; d < hd; d += NT) {
                float kv = p.use_rope ? rope_at(raw + G * hd, d, p.half, ct, st) : raw[G * hd + d];
                float vv = raw[(G + 1) * hd + d];
                const uint64_t idx = (uint64_t)cur * kv_stride + (uint64_t)kvh * hd + d;
                if (p.kv_f16) {
                    const uint16_t kh = f2h(kv), vh = f2h(vv);
                    reinterpret_cast<uint16_t*>(p.kc)[idx] = kh;
                    reinterpret_cast<uint16_t*>(p.vc)[idx] = vh;
                    kv = h2f(kh);   // use the stored value, as later steps will
                    vv = h2f(vh);
                } else {
                    reinterpret_cast<float*>(p.kc)[idx] = kv;
                    reinterpret_cast<float*>(p.vc)[idx] = vv;
                }
                knew[d] = kv;
                vnew[d] = vv;
            }
    } else {
        for (uint32_t i = t; i < G * hd; i += NT) qs[i] = p.q[(uint64_t)kvh * G * hd + i];
    }
    __syncthreads();

    const uint32_t g = (uint32_t)wave;
    if (g >= G) return;
    const float* qg = qs + g * hd;
    const uint32_t hh = hd / 2;                      // dims per half for q.k
    const uint32_t half_id = (uint32_t)lane / 32, r_lane = (uint32_t)lane % 32;
    const uint32_t dq0 = half_id * hh;
    const uint32_t dv0 = (uint32_t)lane * DPL;       // dims of this lane for p.V
    const bool vlane = dv0 < hd;
    float m = -INFINITY, l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;

    for (uint32_t c0 = p0; c0 < p1; c0 += SUB) {
        const uint32_t cn = min((uint32_t)SUB, p1 - c0);
        // V rows of this pass (independent of the scores: issue first)
        float vr[SUB][DPL];
#pragma unroll
        for (int r = 0; r < SUB; ++r) {
            const uint32_t ps = c0 + (uint32_t)r;
            if ((uint32_t)r < cn && vlane) {
                if (has_new && ps == cur) {
#pragma unroll
                    for (int i = 0; i < DPL; ++i) vr[r][i] = vnew[dv0 + i];
                } else {
                    load_v_row<DPL>(p, (uint64_t)ps * kv_stride + (uint64_t)kvh * hd + dv0, vr[r]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < DPL; ++i) vr[r][i] = 0.f;
            }
        }
        // q.k for position c0 + r_lane over dims [dq0, dq0 + hh)
        float s = 0.f;
        const uint32_t ps = c0 + r_lane;
        if (r_lane < cn) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            if (has_new && ps == cur) {
                for (uint32_t d = 0; d < hh; d += 4) {
                    a0 = fmaf(qg[dq0 + d], knew[dq0 + d], a0);
                    a1 = fmaf(qg[dq0 + d + 1], knew[dq0 + d + 1], a1);
                    a2 = fmaf(qg[dq0 + d + 2], knew[dq0 + d + 2], a2);
                    a3 = fmaf(qg[dq0 + d + 3], knew[dq0 + d + 3], a3);
                }
            } else {
                const uint64_t base = (uint64_t)ps * kv_stride + (uint64_t)kvh * hd + dq0;
                if (p.kv_f16) {
                    const uint16_t* kr = reinterpret_cast<const uint16_t*>(p.kc) + base;
                    for (uint32_t d = 0; d < hh; d += 4) {
                        const uint2 w = *reinterpret_cast<const uint2*>(kr + d);
                        a0 = fmaf(qg[dq0 + d], h2f((uint16_t)(w.x & 0xFFFFu)), a0);
                        a1 = fmaf(qg[dq0 + d + 1], h2f((uint16_t)(w.x >> 16)), a1);
                        a2 = fmaf(qg[dq0 + d + 2], h2f((uint16_t)(w.y & 0xFFFFu)), a2);
                        a3 = fmaf(qg[dq0 + d + 3], h2f((uint16_t)(w.y >> 16)), a3);
                    }
                } else {
                    const float* kr = reinterpret_cast<const float*>(p.kc) + base;
                    for (uint32_t d = 0; d < hh; d += 4) {
                        const float4 w = *reinterpret_cast<const float4*>(kr + d);
                        a0 = fmaf(qg[dq0 + d], w.x, a0);
                        a1 = fmaf(qg[dq0 + d + 1], w.y, a1);
                        a2 = fmaf(qg[dq0 + d + 2], w.z, a2);
                        a3 = fmaf(qg[dq0 + d + 3], w.w, a3);
                    }
                }
            }
            s = (a0 + a1) + (a2 + a3);
        }
        s += __shfl_xor(s, 32, kWave);
        s = (r_lane < cn) ? s * p.scale : -INFINITY;
        // online softmax over the pass (lanes r and r + 32 hold the same score)
        const float m_new = fmaxf(m, wave_max(s));
        const float f = expf(m - m_new);          // 0 on the first pass
        const float e = (r_lane < cn) ? expf(s - m_new) : 0.f;
        l = l * f + wave_sum(half_id == 0 ? e : 0.f);
        m = m_new;
        if (half_id == 0) es[g * SUB + r_lane] = e;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] *= f;
#pragma unroll
        for (int r = 0; r < SUB; ++r) {
            const float er = es[g * SUB + r];     // zero beyond cn
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[i] = fmaf(er, vr[r][i], acc[i]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float* part = p.part + (((uint64_t)kvh * p.s_max + split) * G + g) * (hd + 2);
    if (vlane) {
#pragma unroll
        for (int i = 0; i < DPL; ++i)
            if (dv0 + i < hd) part[dv0 + i] = acc[i];
    }
    if (lane == 0) {
        part[hd] = m;
        part[hd + 1] = l;
    }
}

// Merge of the split partials into the attention output, one block per
// query head: out = sum_s acc_s e^(m_s - m) / sum_s l_s e^(m_s - m).
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnCombineParams p) {
    __shared__ float w[kAttnMaxSplits];
    __shared__ float s_inv;
    const uint32_t h = blockIdx.x;
    const uint32_t hd = p.hd, G = p.groups, kvh = h / G, g = h % G;
    const uint32_t L = p.pos ? (uint32_t)(*p.pos) + 1u : p.L;
    const uint32_t s_act = min(p.s_max, (L + p.chunk - 1) / p.chunk);
    const float* base = p.part + ((uint64_t)kvh * p.s_max * G + g) * (hd + 2);
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        float m = -INFINITY;
        for (uint32_t s = lane; s < s_act; s += kWave) m = fmaxf(m, base[(uint64_t)s * G * (hd + 2) + hd]);
        m = wave_max(m);
        float den = 0.f;
        for (uint32_t s = lane; s < s_act; s += kWave) {
            const float* ps = base + (uint64_t)s * G * (hd + 2);
            const float e = expf(ps[hd] - m);
            w[s] = e;
            den += ps[hd + 1] * e;
        }
        den = wave_sum(den);
        if (lane == 0) s_inv = 1.0f / den;
    }
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float v = 0.f;
        for (uint32_t s = 0; s < s_act; ++s) v = fmaf(base[(uint64_t)s * G * (hd + 2) + d], w[s] * s_inv, v);
        p.out[(uint64_t)h * hd + d] = v;
    }
}

// ---------------------------------------------------------------------------
// Embedding row (embed_lookup, gemv.rs:515-526, 710-736): the fixed-point
// residual stream is set to dequant(E[tok]). The token is read on the
// device: tok = src[idx ? *idx : 0].
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
        p.xacc[j] = to_fixed(v);
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
