// Decode-step kernels other than the GEMVs: GQA decode attention over the
// device KV cache, embedding row lookup, and standalone RMSNorm / RoPE /
// argmax used by the kernel-level entry points.
#pragma once

#include <type_traits>

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

// Cache element (pos, kvh, d) at pos * ps + kvh * hs + d: the layout the
// caller declares (AttnParams::kv_ps / kv_hs), token-major by default.
__device__ __forceinline__ uint64_t kv_pos_stride(const AttnParams& p) {
    return p.kv_ps ? p.kv_ps : (uint64_t)p.KVH * p.hd;
}
__device__ __forceinline__ uint64_t kv_head_off(const AttnParams& p, uint32_t kvh) {
    return (uint64_t)kvh * (p.kv_ps ? p.kv_hs : (uint64_t)p.hd);
}

// RoPE partner of dim d (rotate_half over the first 2*half dims,
// apply_rope_raw gemv.rs:869-887): rotated = v[d] * c + sgn * v[partner] * s,
// with c, s the table entries of dim d mod half. Dims past 2*half pass
// through (partner = d, s = 0).
__device__ __forceinline__ uint32_t rope_partner(uint32_t d, uint32_t half) {
    return d < half ? d + half : (d < 2 * half ? d - half : d);
}

// K and V float4s of one 32-position tile held by one thread (thread t of the
// 256-thread subgroup takes float4 e = t + 256*j of the [32][head_dim/4] tile).
template <int TL>
struct KvTileRegs {
    float4 k[TL], v[TL];
};

template <int TL, bool F16KV>
__device__ __forceinline__ KvTileRegs<TL> attn_load_tile(const AttnParams& p, uint32_t t, uint32_t c0, uint32_t L,
                                                          uint64_t pos_stride, uint64_t head_base, uint32_t q4_row,
                                                          uint32_t tile_n) {
    KvTileRegs<TL> r;
#pragma unroll
    for (int j = 0; j < TL; ++j) {
        const uint32_t e = min(t + (uint32_t)(256 * j), tile_n - 1u);
        const uint32_t row = e / q4_row, c4 = e % q4_row;
        const uint32_t pos = min(c0 + row, L - 1u);
        const uint64_t idx = (uint64_t)pos * pos_stride + head_base + 4u * c4;
        if constexpr (F16KV) {
            const uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.kc) + idx);
            const uint2 b = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.vc) + idx);
            r.k[j] = make_float4(h2f((uint16_t)(a.x & 0xFFFFu)), h2f((uint16_t)(a.x >> 16)),
                                 h2f((uint16_t)(a.y & 0xFFFFu)), h2f((uint16_t)(a.y >> 16)));
            r.v[j] = make_float4(h2f((uint16_t)(b.x & 0xFFFFu)), h2f((uint16_t)(b.x >> 16)),
                                 h2f((uint16_t)(b.y & 0xFFFFu)), h2f((uint16_t)(b.y >> 16)));
        } else {
            r.k[j] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.kc) + idx);
            r.v[j] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.vc) + idx);
        }
    }
    return r;
}

// Rows at or past cn become zeros (a bit mask, not a select: exact zeros
// whatever stale bits the unwritten slots hold); row `skip` (the appended
// position, or >= 32 for none) is left to its writer.
template <int TL, int KSTR, int VSTR>
__device__ __forceinline__ void attn_store_tile(const KvTileRegs<TL>& r, uint32_t t, float* ktile, float* vtile,
                                                uint32_t cn, uint32_t skip, uint32_t q4_row, uint32_t tile_n) {
#pragma unroll
    for (int j = 0; j < TL; ++j) {
        const uint32_t e = t + (uint32_t)(256 * j);
        const uint32_t row = e / q4_row, c4 = e % q4_row;
        if (e < tile_n && row != skip) {
            const uint32_t msk = row < cn ? 0xFFFFFFFFu : 0u;
            const uint4 kb = make_uint4(__float_as_uint(r.k[j].x) & msk, __float_as_uint(r.k[j].y) & msk,
                                        __float_as_uint(r.k[j].z) & msk, __float_as_uint(r.k[j].w) & msk);
            const uint4 vb = make_uint4(__float_as_uint(r.v[j].x) & msk, __float_as_uint(r.v[j].y) & msk,
                                        __float_as_uint(r.v[j].z) & msk, __float_as_uint(r.v[j].w) & msk);
            *reinterpret_cast<uint4*>(ktile + row * KSTR + 4 * c4) = kb;
            *reinterpret_cast<uint4*>(vtile + row * VSTR + 4 * c4) = vb;
        }
    }
}

// Block (split, kvh) walks its positions in passes of 32. Each pass's K and
// V rows are loaded once per block with coalesced 16-byte loads (256 lanes,
// 4 KB per instruction) and staged in LDS as fp32; rows past the pass are
// stored as zeros. The next pass is prefetched into registers while the
// current one is computed. One wave per query head then takes its scores
// from the K tile (lanes (half, r) = (lane / 32, lane % 32): position r,
// half of the dims), runs the online softmax and accumulates p.V from the V
// tile (DPL dims per lane). In model mode the appended position's K/V row
// is computed here (RMSNorm factor, RoPE), written to the cache and put
// into the tile directly.
// Latency: the loads that do not depend on the position (q|k|v sums,
// RMSNorm partials) are issued together with the position load; the cache
// tile and RoPE tables follow as soon as the position arrives. q and the K
// rows are zero-padded to HDM dims in LDS so the dot products run without
// predicates. DPL = 2 covers head_dim <= 128, DPL = 1 head_dim <= 64.
// chunk = p.chunk, or attn_chunk_for(L) when 0 (the split count then stays
// within kAttnMaxSplits at every context length). Contexts whose splits hold
// many passes take attn_decode_long_kernel instead.
template <int DPL, bool F16KV>
__global__ __launch_bounds__(256) void attn_decode_kernel(const int32_t* pos_p, const long long* qkv,
                                                          const float* ssin, const float* rcos, const float* rsin,
                                                          uint32_t shape, uint32_t hh, uint32_t snn, uint32_t chunk_a,
                                                          AttnParams p) {
    // (first-load arguments preloaded; see launch_attn)
    const uint32_t half = (hh >> 16) & 0x7FFFu, H = hh & 0xFFFFu, KVH = shape >> 20;
    const bool use_rope = (hh >> 31) != 0u;
    const uint32_t ss_n = snn & 0xFFu, norm_n = snn >> 8;
    constexpr int NT = 256;
    constexpr int SUB = kAttnSub;                    // positions per pass (32)
    constexpr int HDM = 64 * DPL;                    // head_dim bound of this instance
    constexpr int KQ = HDM / 8;                      // float4 chunks per lane for q.k (half of HDM)
    constexpr int KSTR = HDM + 4;                    // padded K row stride (floats): no bank conflicts
    constexpr int VSTR = HDM;
    constexpr int TL = SUB * HDM / 4 / NT;           // float4 per thread per tile
    __shared__ __align__(16) float ktile[SUB * KSTR];
    __shared__ __align__(16) float vtile[SUB * VSTR];
    __shared__ __align__(16) float qs[kAttnMaxGroups * HDM];
    __shared__ float es[kAttnMaxGroups * SUB];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t hd = shape & 0x3FFu, G = (shape >> 10) & 0x3FFu;
    const bool model = qkv != nullptr;
    const uint64_t kv_stride = (uint64_t)KVH * hd;    // q|k|v accumulator layout
    const uint64_t head_off = (uint64_t)kvh * hd;
    const uint64_t cps = p.kv_ps ? p.kv_ps : kv_stride, coff = (uint64_t)kvh * (p.kv_ps ? p.kv_hs : (uint64_t)hd);   // cache layout
    const uint32_t nq = G * hd;

    // ---- position-independent loads, in flight with the position (a scalar
    // load: waiting for it does not wait for the vector loads) ----
    const int32_t pos_raw = pos_p ? ld_scalar_i32(pos_p) : (int32_t)p.L - 1;
    long long qa[2] = {0, 0}, qb[2] = {0, 0};
    long long ka = 0, kb = 0, va = 0;
    float ssp = 0.f;
    const uint32_t dn = min((uint32_t)t, hd - 1u);
    if (model) {
        const uint32_t qd = H * hd;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t i = min((uint32_t)t + (uint32_t)u * NT, nq - 1u);
            const uint32_t d = i % hd;
            qa[u] = qkv[(uint64_t)kvh * G * hd + i];
            qb[u] = qkv[(uint64_t)kvh * G * hd + (i - d) + rope_partner(d, half)];
        }
        ka = qkv[qd + head_off + dn];
        kb = qkv[qd + head_off + rope_partner(dn, half)];
        va = qkv[qd + kv_stride + head_off + dn];
        ssp = ssin[min((uint32_t)lane, ss_n - 1u)];
    }

    const uint32_t L = (uint32_t)pos_raw + 1u;
    const uint32_t chunk = chunk_a ? chunk_a : attn_chunk_for(L);
    const uint32_t p0 = split * chunk;
    if (p0 >= L) {
        // the loads above are used on this path too, so the compiler issues
        // them before the position is known instead of sinking them past
        // this branch (behind a wait for the position)
        asm volatile("" ::"v"(qa[0]), "v"(qa[1]), "v"(qb[0]), "v"(qb[1]), "v"(ka), "v"(kb), "v"(va), "v"(ssp));
        return;
    }
    const uint32_t p1 = min(L, p0 + chunk);
    const uint32_t cur = L - 1;                        // position appended this step
    const bool has_new = model && cur >= p0 && cur < p1;
    const uint32_t q4_row = hd / 4;                    // float4 per row
    const uint32_t tile_n = SUB * q4_row;              // float4 per tile

    // ---- position-dependent loads: RoPE entries of `cur`, first cache tile ----
    float qc[2] = {1.f, 1.f}, qsn[2] = {0.f, 0.f}, kc_ = 1.f, ks_ = 0.f;
    if (model && use_rope) {
        const float* ct = rcos + (uint64_t)cur * half;
        const float* st = rsin + (uint64_t)cur * half;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t d = min((uint32_t)t + (uint32_t)u * NT, nq - 1u) % hd;
            const uint32_t td = d < half ? d : (d < 2 * half ? d - half : 0u);
            qc[u] = ct[td];
            qsn[u] = st[td];
        }
        const uint32_t td = dn < half ? dn : (dn < 2 * half ? dn - half : 0u);
        kc_ = ct[td];
        ks_ = st[td];
    }
    KvTileRegs<TL> tr = attn_load_tile<TL, F16KV>(p, threadIdx.x, p0, L, cps, coff, q4_row, tile_n);

    // K padding columns [hd, HDM) stay zero for the whole kernel
    if (hd < (uint32_t)HDM)
        for (uint32_t e = t; e < SUB * ((uint32_t)HDM - hd); e += NT)
            ktile[(e / ((uint32_t)HDM - hd)) * KSTR + hd + e % ((uint32_t)HDM - hd)] = 0.f;

    // ---- q of the group's heads (and the appended k, v) ----
    float k_app = 0.f, v_app = 0.f;                   // thread t < hd: dim t of the appended row
    if (model) {
        // the q|k|v GEMV ran on x * gamma; its RMSNorm factor is applied here
        const float inv = 1.0f / sqrtf(wave_sum(lane < (int)ss_n ? ssp : 0.f) / (float)norm_n + 1e-6f);
        const bool rot = use_rope != 0;
        // padding dims [hd, HDM) of each q row are zero
        for (uint32_t i = t; i < G * HDM; i += NT)
            if (i % HDM >= hd) qs[i] = 0.f;
        // q values: thread t owns flat index i = t + 256u of [G][hd]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t i = (uint32_t)t + (uint32_t)u * NT;
            if (i < nq) {
                const uint32_t d = i % hd;
                const float a = inv * from_fixed(qa[u]), b = inv * from_fixed(qb[u]);
                // rotate_half: the first half takes -partner * sin, the second +partner * sin
                qs[(i / hd) * HDM + d] = (rot && d < 2 * half) ? (d < half ? a * qc[u] - b * qsn[u]
                                                                                 : a * qc[u] + b * qsn[u])
                                                                  : a;
            }
        }
        if (has_new && (uint32_t)t < hd) {
            const float a = inv * from_fixed(ka), b = inv * from_fixed(kb);
            float kv = (rot && dn < 2 * half) ? (dn < half ? a * kc_ - b * ks_ : a * kc_ + b * ks_) : a;
            float vv = inv * from_fixed(va);
            const uint64_t idx = (uint64_t)cur * cps + coff + dn;
            if constexpr (F16KV) {
                const uint16_t kh = f2h(kv), vh = f2h(vv);
                reinterpret_cast<uint16_t*>(p.kc)[idx] = kh;
                reinterpret_cast<uint16_t*>(p.vc)[idx] = vh;
                kv = h2f(kh);   // use the stored value, as later steps will
                vv = h2f(vh);
            } else {
                reinterpret_cast<float*>(p.kc)[idx] = kv;
                reinterpret_cast<float*>(p.vc)[idx] = vv;
            }
            k_app = kv;
            v_app = vv;
        }
    } else {
        for (uint32_t i = t; i < G * HDM; i += NT) {
            const uint32_t g = i / HDM, d = i % HDM;
            qs[i] = d < hd ? p.q[(uint64_t)(kvh * G + g) * hd + d] : 0.f;
        }
    }

    const uint32_t g = (uint32_t)wave;
    const uint32_t half_id = (uint32_t)lane / 32, r_lane = (uint32_t)lane % 32;
    const uint32_t dq0 = half_id * (HDM / 2);
    const uint32_t dv0c = min((uint32_t)lane * DPL, hd - DPL);   // clamped V dims of this lane
    const bool vlane = (uint32_t)lane * DPL < hd;
    float m = -INFINITY, l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;

    for (uint32_t c0 = p0; c0 < p1; c0 += SUB) {
        const uint32_t cn = min((uint32_t)SUB, p1 - c0);
        const bool new_here = has_new && cur >= c0 && cur < c0 + cn;
        attn_store_tile<TL, KSTR, VSTR>(tr, threadIdx.x, ktile, vtile, cn, new_here ? cur - c0 : 0xFFFFFFFFu, q4_row, tile_n);
        if (new_here && (uint32_t)t < hd) {
            ktile[(cur - c0) * KSTR + t] = k_app;
            vtile[(cur - c0) * VSTR + t] = v_app;
        }
        __syncthreads();
        if (c0 + SUB < p1)                            // next pass, in flight during this one
            tr = attn_load_tile<TL, F16KV>(p, threadIdx.x, c0 + SUB, L, cps, coff, q4_row, tile_n);
        if (g < G) {
            // q.k for position c0 + r_lane over padded dims [dq0, dq0 + HDM/2)
            const float* qg = qs + g * HDM + dq0;
            const float* krow = ktile + r_lane * KSTR + dq0;
            float4 q4[KQ], k4[KQ];
#pragma unroll
            for (int i = 0; i < KQ; ++i) {
                q4[i] = *reinterpret_cast<const float4*>(qg + 4 * i);
                k4[i] = *reinterpret_cast<const float4*>(krow + 4 * i);
            }
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int i = 0; i < KQ; ++i) {
                a0 = fmaf(q4[i].x, k4[i].x, a0);
                a1 = fmaf(q4[i].y, k4[i].y, a1);
                a2 = fmaf(q4[i].z, k4[i].z, a2);
                a3 = fmaf(q4[i].w, k4[i].w, a3);
            }
            float s = (a0 + a1) + (a2 + a3);
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
            // rows past the pass are zeros in the tile and have zero weight
#pragma unroll
            for (int r = 0; r < SUB; ++r) {
                const float er = es[g * SUB + r];
                const float* vrow = vtile + r * VSTR + dv0c;
                if constexpr (DPL == 2) {
                    const float2 v2 = *reinterpret_cast<const float2*>(vrow);
                    acc[0] = fmaf(er, v2.x, acc[0]);
                    acc[1] = fmaf(er, v2.y, acc[1]);
                } else {
                    acc[0] = fmaf(er, vrow[0], acc[0]);
                }
            }
        }
        __syncthreads();                              // the tile is rewritten next pass
    }
    if (g >= G) return;
    float* part = p.part + (((uint64_t)kvh * p.s_max + split) * G + g) * (hd + 2);
    if (vlane) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) part[dv0c + i] = acc[i];
    }
    if (lane == 0) {
        part[hd] = m;
        part[hd + 1] = l;
    }
}

// Raw cache words of one 32-position tile as loaded (binary16 quads or fp32
// float4s), converted to fp32 only when stored to LDS: an f16 tile then costs
// 16 VGPRs instead of 32, so two tiles can be in flight per subgroup.
template <int TL, bool F16KV>
struct KvRaw {
    using W = typename std::conditional<F16KV, uint2, float4>::type;
    W k[TL], v[TL];
};

template <int TL, bool F16KV>
__device__ __forceinline__ void attn_load_raw(KvRaw<TL, F16KV>& r, const AttnParams& p, uint32_t t, uint32_t c0,
                                              uint32_t L, uint64_t pos_stride, uint64_t head_base, uint32_t q4_row,
                                              uint32_t tile_n) {
    using W = typename KvRaw<TL, F16KV>::W;
    constexpr uint32_t wb = F16KV ? 2u : 4u;   // bytes per element
#pragma unroll
    for (int j = 0; j < TL; ++j) {
        const uint32_t e = min(t + (uint32_t)(256 * j), tile_n - 1u);
        const uint32_t row = e / q4_row, c4 = e % q4_row;
        const uint32_t pos = min(c0 + row, L - 1u);
        const uint64_t off = ((uint64_t)pos * pos_stride + head_base + 4u * c4) * wb;
        r.k[j] = *reinterpret_cast<const W*>(reinterpret_cast<const uint8_t*>(p.kc) + off);
        r.v[j] = *reinterpret_cast<const W*>(reinterpret_cast<const uint8_t*>(p.vc) + off);
    }
}

__device__ __forceinline__ float4 kv_words_f32(uint2 a) {
    return make_float4(h2f((uint16_t)(a.x & 0xFFFFu)), h2f((uint16_t)(a.x >> 16)), h2f((uint16_t)(a.y & 0xFFFFu)),
                       h2f((uint16_t)(a.y >> 16)));
}
__device__ __forceinline__ float4 kv_words_f32(float4 a) { return a; }

// As attn_store_tile, from raw words.
template <int TL, bool F16KV, int KSTR, int VSTR>
__device__ __forceinline__ void attn_store_raw(const KvRaw<TL, F16KV>& r, uint32_t t, float* ktile, float* vtile,
                                               uint32_t cn, uint32_t skip, uint32_t q4_row, uint32_t tile_n) {
#pragma unroll
    for (int j = 0; j < TL; ++j) {
        const uint32_t e = t + (uint32_t)(256 * j);
        const uint32_t row = e / q4_row, c4 = e % q4_row;
        if (e < tile_n && row != skip) {
            const uint32_t msk = row < cn ? 0xFFFFFFFFu : 0u;
            const float4 kf = kv_words_f32(r.k[j]), vf = kv_words_f32(r.v[j]);
            const uint4 kb = make_uint4(__float_as_uint(kf.x) & msk, __float_as_uint(kf.y) & msk,
                                        __float_as_uint(kf.z) & msk, __float_as_uint(kf.w) & msk);
            const uint4 vb = make_uint4(__float_as_uint(vf.x) & msk, __float_as_uint(vf.y) & msk,
                                        __float_as_uint(vf.z) & msk, __float_as_uint(vf.w) & msk);
            *reinterpret_cast<uint4*>(ktile + row * KSTR + 4 * c4) = kb;
            *reinterpret_cast<uint4*>(vtile + row * VSTR + 4 * c4) = vb;
        }
    }
}

// Long contexts: the same computation with each block's passes split among
// NSG = 4 subgroups of 256 threads (subgroup sg takes passes sg, sg + NSG, ...).
// Each pass's K and V rows are loaded once with coalesced 16-byte loads
// (256 lanes, 4 KB per instruction) and staged in the subgroup's LDS tiles as
// fp32; rows past the pass are stored as zeros. The subgroup's next pass is
// prefetched into registers (raw cache words) while the current one is
// computed, so 4 tiles per block are in flight: a split of a long context
// holds many passes, and one tile in flight per block leaves HBM idle. One wave per
// query head then takes its scores from the K tile (lanes (half, r) =
// (lane / 32, lane % 32): position r, half of the dims), runs the online
// softmax and accumulates p.V from the V tile (DPL dims per lane). The
// subgroups' (max, sum, p.V) states are merged in LDS, in subgroup order.
// In model mode the appended position's K/V row is computed here (RMSNorm
// factor, RoPE), written to the cache and put into the tile directly.
// Latency: the loads that do not depend on the position (q|k|v sums,
// RMSNorm partials) are issued together with the position load; the cache
// tile and RoPE tables follow as soon as the position arrives. q and the K
// rows are zero-padded to HDM dims in LDS so the dot products run without
// predicates. DPL = 2 covers head_dim <= 128, DPL = 1 head_dim <= 64.
// chunk = p.chunk, or attn_chunk_for(L) when 0 (the split count then stays
// within kAttnMaxSplits at every context length).
constexpr int kAttnLongNsg = 4;

template <int DPL, bool F16KV>
__global__ __launch_bounds__(256 * kAttnLongNsg) void attn_decode_long_kernel(AttnParams p) {
    kernarg_warm(p);
    constexpr int NSG = kAttnLongNsg;
    constexpr int NT = 256;                          // threads per subgroup
    constexpr int SUB = kAttnSub;                    // positions per pass (32)
    constexpr int HDM = 64 * DPL;                    // head_dim bound of this instance
    constexpr int KQ = HDM / 8;                      // float4 chunks per lane for q.k (half of HDM)
    constexpr int KSTR = HDM + 4;                    // padded K row stride (floats): no bank conflicts
    constexpr int VSTR = HDM;
    constexpr int TL = SUB * HDM / 4 / NT;           // float4 per thread per tile
    constexpr int QC = 4;
    static_assert(NSG * SUB * KSTR >= NSG * kAttnMaxGroups * HDM, "merge scratch must fit in the K tiles");
    __shared__ __align__(16) float ktile[NSG][SUB * KSTR];
    __shared__ __align__(16) float vtile[NSG][SUB * VSTR];
    __shared__ __align__(16) float qs[kAttnMaxGroups * HDM];
    __shared__ float es[NSG][kAttnMaxGroups * SUB];
    __shared__ float knew[HDM], vnew[HDM];
    __shared__ float red_m[NSG][kAttnMaxGroups], red_l[NSG][kAttnMaxGroups];

    const int t = (int)(threadIdx.x % NT);           // thread within the subgroup
    // wave-uniform (a scalar register), so the pass bookkeeping stays scalar
    const int sg = __builtin_amdgcn_readfirstlane(threadIdx.x / NT);
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t hd = p.hd, G = p.groups;
    const bool model = p.qkv_acc != nullptr;
    const bool lead = sg == 0;                       // subgroup 0 sets up q and the appended row
    const uint64_t kv_stride = (uint64_t)p.KVH * hd;    // q|k|v accumulator layout
    const uint64_t head_off = (uint64_t)kvh * hd;
    const uint64_t cps = kv_pos_stride(p), coff = kv_head_off(p, kvh);   // cache layout
    const uint32_t nq = G * hd;

    // ---- position-independent loads, in flight with the position (a scalar
    // load: waiting for it does not wait for the vector loads) ----
    const int32_t pos_raw = p.pos ? ld_scalar_i32(p.pos) : (int32_t)p.L - 1;
    long long qa[2] = {0, 0}, qb[2] = {0, 0};
    long long ka = 0, kb = 0, va = 0;
    float ssp = 0.f;
    const uint32_t dn = min((uint32_t)t, hd - 1u);
    if (model && lead) {
        const uint32_t qd = p.H * hd;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t i = min((uint32_t)t + (uint32_t)u * NT, nq - 1u);
            const uint32_t d = i % hd;
            qa[u] = p.qkv_acc[(uint64_t)kvh * G * hd + i];
            qb[u] = p.qkv_acc[(uint64_t)kvh * G * hd + (i - d) + rope_partner(d, p.half)];
        }
        ka = p.qkv_acc[qd + head_off + dn];
        kb = p.qkv_acc[qd + head_off + rope_partner(dn, p.half)];
        va = p.qkv_acc[qd + kv_stride + head_off + dn];
        ssp = p.ss_in[min((uint32_t)lane, p.ss_n - 1u)];
    }

    const uint32_t L = (uint32_t)pos_raw + 1u;
    const uint32_t chunk = p.chunk ? p.chunk : attn_chunk_for(L);
    const uint32_t p0 = split * chunk;
    if (p0 >= L) {                                     // whole block: no barrier reached yet
        // used on this path too: the loads above go out before the position
        asm volatile("" ::"v"(qa[0]), "v"(qa[1]), "v"(qb[0]), "v"(qb[1]), "v"(ka), "v"(kb), "v"(va), "v"(ssp));
        return;
    }
    const uint32_t p1 = min(L, p0 + chunk);
    const uint32_t cur = L - 1;                        // position appended this step
    const bool has_new = model && cur >= p0 && cur < p1;
    const uint32_t q4_row = hd / 4;                    // float4 per row
    const uint32_t tile_n = SUB * q4_row;              // float4 per tile
    const uint32_t npass = (p1 - p0 + SUB - 1) / SUB;
    const uint32_t iters = (npass + NSG - 1) / NSG;

    // ---- position-dependent loads: RoPE entries of `cur`, first cache tile ----
    float qc[2] = {1.f, 1.f}, qsn[2] = {0.f, 0.f}, kc_ = 1.f, ks_ = 0.f;
    if (model && lead && p.use_rope) {
        const float* ct = p.rope_cos + (uint64_t)cur * p.half;
        const float* st = p.rope_sin + (uint64_t)cur * p.half;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t d = min((uint32_t)t + (uint32_t)u * NT, nq - 1u) % hd;
            const uint32_t td = d < p.half ? d : (d < 2 * p.half ? d - p.half : 0u);
            qc[u] = ct[td];
            qsn[u] = st[td];
        }
        const uint32_t td = dn < p.half ? dn : (dn < 2 * p.half ? dn - p.half : 0u);
        kc_ = ct[td];
        ks_ = st[td];
    }
    // passes in flight per subgroup; 2 (an f16 tile is 16 VGPRs raw) measured
    // no faster at 32768 positions: the LDS traffic of the q.k and p.V loops,
    // not HBM latency, is then what bounds the kernel
    constexpr int DEPTH = 1;
    KvRaw<TL, F16KV> tr[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if ((uint32_t)sg + (uint32_t)(d * NSG) < npass)
            attn_load_raw<TL, F16KV>(tr[d], p, t, p0 + ((uint32_t)sg + (uint32_t)(d * NSG)) * SUB, L, cps, coff,
                                     q4_row, tile_n);

    // K padding columns [hd, HDM) stay zero for the whole kernel
    if (hd < (uint32_t)HDM)
        for (uint32_t e = t; e < SUB * ((uint32_t)HDM - hd); e += NT)
            ktile[sg][(e / ((uint32_t)HDM - hd)) * KSTR + hd + e % ((uint32_t)HDM - hd)] = 0.f;

    // ---- q of the group's heads (and the appended k, v) ----
    if (model && lead) {
        // the q|k|v GEMV ran on x * gamma; its RMSNorm factor is applied here
        const float inv = 1.0f / sqrtf(wave_sum(lane < (int)p.ss_n ? ssp : 0.f) / (float)p.norm_n + 1e-6f);
        const bool rot = p.use_rope != 0;
        // padding dims [hd, HDM) of each q row are zero
        for (uint32_t i = t; i < G * HDM; i += NT)
            if (i % HDM >= hd) qs[i] = 0.f;
        // q values: thread t owns flat index i = t + 256u of [G][hd]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t i = (uint32_t)t + (uint32_t)u * NT;
            if (i < nq) {
                const uint32_t d = i % hd;
                const float a = inv * from_fixed(qa[u]), b = inv * from_fixed(qb[u]);
                // rotate_half: the first half takes -partner * sin, the second +partner * sin
                qs[(i / hd) * HDM + d] = (rot && d < 2 * p.half) ? (d < p.half ? a * qc[u] - b * qsn[u]
                                                                                 : a * qc[u] + b * qsn[u])
                                                                  : a;
            }
        }
        if (has_new && (uint32_t)t < hd) {
            const float a = inv * from_fixed(ka), b = inv * from_fixed(kb);
            float kv = (rot && dn < 2 * p.half) ? (dn < p.half ? a * kc_ - b * ks_ : a * kc_ + b * ks_) : a;
            float vv = inv * from_fixed(va);
            const uint64_t idx = (uint64_t)cur * cps + coff + dn;
            if constexpr (F16KV) {
                const uint16_t kh = f2h(kv), vh = f2h(vv);
                reinterpret_cast<uint16_t*>(p.kc)[idx] = kh;
                reinterpret_cast<uint16_t*>(p.vc)[idx] = vh;
                kv = h2f(kh);   // use the stored value, as later steps will
                vv = h2f(vh);
            } else {
                reinterpret_cast<float*>(p.kc)[idx] = kv;
                reinterpret_cast<float*>(p.vc)[idx] = vv;
            }
            knew[t] = kv;
            vnew[t] = vv;
        }
    } else if (lead) {
        for (uint32_t i = t; i < G * HDM; i += NT) {
            const uint32_t g = i / HDM, d = i % HDM;
            qs[i] = d < hd ? p.q[(uint64_t)(kvh * G + g) * hd + d] : 0.f;
        }
    }
    __syncthreads();                                 // qs, knew, vnew

    const uint32_t g = (uint32_t)wave;
    const uint32_t half_id = (uint32_t)lane / 32, r_lane = (uint32_t)lane % 32;
    const uint32_t dq0 = half_id * (HDM / 2);
    const uint32_t dv0c = min((uint32_t)lane * DPL, hd - DPL);   // clamped V dims of this lane
    const bool vlane = (uint32_t)lane * DPL < hd;
    float* kt = ktile[sg];
    float* vt = vtile[sg];
    float* et = es[sg];
    float m = -INFINITY, l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;

    // one pass of this subgroup, from the raw tile `rt` (refilled with the pass
    // DEPTH rounds ahead once its words are in LDS)
    auto pass = [&](KvRaw<TL, F16KV>& rt, uint32_t it) {
        const uint32_t pi = it * NSG + (uint32_t)sg;   // this subgroup's pass
        const bool active = pi < npass;
        const uint32_t c0 = p0 + pi * SUB;
        const uint32_t cn = active ? min((uint32_t)SUB, p1 - c0) : 0u;
        if (active) {
            const bool new_here = has_new && cur >= c0 && cur < c0 + cn;
            attn_store_raw<TL, F16KV, KSTR, VSTR>(rt, t, kt, vt, cn, new_here ? cur - c0 : 0xFFFFFFFFu, q4_row, tile_n);
            if (new_here && (uint32_t)t < hd) {
                kt[(cur - c0) * KSTR + t] = knew[t];
                vt[(cur - c0) * VSTR + t] = vnew[t];
            }
        }
        __syncthreads();
        if (pi + DEPTH * NSG < npass)                  // in flight during the next DEPTH passes
            attn_load_raw<TL, F16KV>(rt, p, t, c0 + DEPTH * NSG * SUB, L, cps, coff, q4_row, tile_n);
        if (active && g < G) {
            // q.k for position c0 + r_lane over padded dims [dq0, dq0 + HDM/2)
            const float* qg = qs + g * HDM + dq0;
            const float* krow = kt + r_lane * KSTR + dq0;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            // QC float4 pairs at a time: the whole row in registers (128 VGPRs)
            // would not fit the 128-VGPR budget of a 1024-thread block
#pragma unroll
            for (int i0 = 0; i0 < KQ; i0 += QC) {
                float4 q4[QC], k4[QC];
#pragma unroll
                for (int i = 0; i < QC; ++i) {
                    q4[i] = *reinterpret_cast<const float4*>(qg + 4 * (i0 + i));
                    k4[i] = *reinterpret_cast<const float4*>(krow + 4 * (i0 + i));
                }
#pragma unroll
                for (int i = 0; i < QC; ++i) {
                    a0 = fmaf(q4[i].x, k4[i].x, a0);
                    a1 = fmaf(q4[i].y, k4[i].y, a1);
                    a2 = fmaf(q4[i].z, k4[i].z, a2);
                    a3 = fmaf(q4[i].w, k4[i].w, a3);
                }
            }
            float s = (a0 + a1) + (a2 + a3);
            s += __shfl_xor(s, 32, kWave);
            s = (r_lane < cn) ? s * p.scale : -INFINITY;
            // online softmax over the pass (lanes r and r + 32 hold the same score)
            const float m_new = fmaxf(m, wave_max(s));
            const float f = expf(m - m_new);          // 0 on the first pass
            const float e = (r_lane < cn) ? expf(s - m_new) : 0.f;
            l = l * f + wave_sum(half_id == 0 ? e : 0.f);
            m = m_new;
            if (half_id == 0) et[g * SUB + r_lane] = e;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[i] *= f;
            // rows past the pass are zeros in the tile and have zero weight
#pragma unroll
            for (int r = 0; r < SUB; ++r) {
                const float er = et[g * SUB + r];
                const float* vrow = vt + r * VSTR + dv0c;
                if constexpr (DPL == 2) {
                    const float2 v2 = *reinterpret_cast<const float2*>(vrow);
                    acc[0] = fmaf(er, v2.x, acc[0]);
                    acc[1] = fmaf(er, v2.y, acc[1]);
                } else {
                    acc[0] = fmaf(er, vrow[0], acc[0]);
                }
            }
        }
        __syncthreads();                              // the tile is rewritten next pass
    };
    for (uint32_t it = 0; it < iters; it += DEPTH) {
        pass(tr[0], it);
        if (DEPTH == 2 && it + 1 < iters) pass(tr[DEPTH - 1], it + 1);
    }
    {
        // merge the subgroups' states (the K tiles are free after the last barrier)
        float* racc = &ktile[0][0];                    // [NSG][G][HDM]
        if (g < G) {
            if (vlane) {
#pragma unroll
                for (int i = 0; i < DPL; ++i) racc[((uint32_t)sg * G + g) * HDM + dv0c + i] = acc[i];
            }
            if (lane == 0) {
                red_m[sg][g] = m;
                red_l[sg][g] = l;
            }
        }
        __syncthreads();
        if (sg != 0 || g >= G) return;
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < NSG; ++j) mx = fmaxf(mx, red_m[j][g]);
        l = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
#pragma unroll
        for (int j = 0; j < NSG; ++j) {
            const float w = expf(red_m[j][g] - mx);     // 0 for a subgroup without passes
            l = fmaf(red_l[j][g], w, l);
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[i] = fmaf(racc[((uint32_t)j * G + g) * HDM + dv0c + i], w, acc[i]);
        }
        m = mx;
    }
    if (g >= G) return;
    float* part = p.part + (((uint64_t)kvh * p.s_max + split) * G + g) * (hd + 2);
    if (vlane) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) part[dv0c + i] = acc[i];
    }
    if (lane == 0) {
        part[hd] = m;
        part[hd + 1] = l;
    }
}

// Long contexts with an f16 cache: no LDS staging of the cache. Block (KV
// head, split) of NWV waves; wave w takes the 8-position passes w, w + NWV,
// ... of the split (short passes keep every wave busy on splits of a few
// hundred positions and the register set small: 8.8% faster decode at 8192
// positions than 32-position passes, 2.8% at 32700). Every lane works on
// the same slice of the row throughout: lane (c, j) = (l % 16, l / 16) holds
// dims [c HD/16, (c + 1) HD/16) of positions 4 i + j (i < 2) of the pass,
// so each K and V load instruction
// reads 4 whole rows (1 KB at HD 128) and a lane's scores are those of the
// very positions whose V it holds: the probabilities never leave the lane.
// Partial dot products are summed over the 16 lanes of a row (4 shuffles),
// the online softmax runs per wave for the G query heads, and the waves'
// (max, sum, p.V) states are merged in wave order at the end. The appended
// row (model mode) comes from LDS, and positions at or past the split's end
// never reach a sum (selection, not a zero weight: stale slots may hold NaN).
template <int HD>
__global__ __launch_bounds__(512) void attn_decode_direct_kernel(const int32_t* pos_a, AttnParams p) {
    // the position's pointer is preloaded into scalar registers at wave
    // launch: its load goes out with the parameter block's lines, and one
    // wait covers both
    const int32_t pos_ld = pos_a ? ld_scalar_i32(pos_a) : 0;
    kernarg_warm(p);
    constexpr int NWV = 8;                           // waves per block
    constexpr int PP = 8;                            // positions per pass (2 rows a lane)
    constexpr int VD = HD / 16;                      // dims per lane
    constexpr int NI = PP / 4;                       // rows per lane per pass
    constexpr int G4 = kAttnMaxGroups;
    typedef typename std::conditional<VD == 8, uint4, uint2>::type VW;
    __shared__ __align__(16) float qs[G4 * HD];
    __shared__ float knew[HD], vnew[HD];
    __shared__ __align__(16) float red_o[NWV][G4][HD];
    __shared__ float red_m[NWV][G4], red_l[NWV][G4];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t % kWave;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t / kWave);
    // grid (KVH, splits)
    const uint32_t kvh = blockIdx.x, split = blockIdx.y;
    const uint32_t hd = HD, G = p.groups;
    const bool model = p.qkv_acc != nullptr;
    const uint64_t kv_stride = (uint64_t)p.KVH * HD;    // q|k|v accumulator layout
    const uint64_t head_off = (uint64_t)kvh * HD;
    const uint64_t cps = kv_pos_stride(p), coff = kv_head_off(p, kvh);   // cache layout

    const int32_t pos_raw = pos_a ? pos_ld : (int32_t)p.L - 1;
    const uint32_t L = (uint32_t)pos_raw + 1u;
    const uint32_t chunk = p.chunk ? p.chunk : attn_chunk_for(L);
    const uint32_t p0 = split * chunk;
    if (p0 >= L) return;                               // whole block: no barrier reached yet
    const uint32_t p1 = min(L, p0 + chunk);
    const uint32_t cur = L - 1;
    const bool has_new = model && cur >= p0 && cur < p1;
    const uint32_t npass = (p1 - p0 + PP - 1) / PP;

    // ---- loads, in the order their data is needed: the q set-up's inputs
    // (threads 0..255), then this wave's first pass of cache rows (they depend
    // on the position only; the row being appended, if read here, is replaced
    // from LDS below), then the q arithmetic waits for its own loads only ----
    const uint32_t vc = lane % 16, vj = lane / 16;    // dim slice, position phase
    const uint16_t* kc = reinterpret_cast<const uint16_t*>(p.kc);
    const uint16_t* vcache = reinterpret_cast<const uint16_t*>(p.vc);
    VW kr[NI], vr[NI];
    auto load_row = [&](VW& dst, const uint16_t* src, uint32_t c0, int i) {
        const uint64_t off = (uint64_t)min(c0 + 4u * i + vj, p1 - 1u) * cps + coff + vc * VD;
        dst = *reinterpret_cast<const VW*>(src + off);
    };
    auto load_rows = [&](VW (&dst)[NI], const uint16_t* src, uint32_t c0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) load_row(dst[i], src, c0, i);
    };
    constexpr uint32_t QPT = G4 * HD / 256;          // q values per set-up thread
    const bool qset = t < 256 && model;
    const uint32_t qd = p.H * hd;
    const bool rot = p.use_rope != 0;
    long long qa[QPT], qb[QPT], ka = 0, kb = 0, va = 0;
    float qc[QPT], qsn[QPT], kc_ = 1.f, ks_ = 0.f, ssp = 0.f;
    if (qset) {
        ssp = p.ss_in[min((uint32_t)lane, p.ss_n - 1u)];
        const float* ct = p.rope_cos + (uint64_t)cur * p.half;
        const float* st = p.rope_sin + (uint64_t)cur * p.half;
#pragma unroll
        for (uint32_t u = 0; u < QPT; ++u) {
            const uint32_t i = min(t + 256u * u, G * hd - 1u), d = i % hd;
            const long long* src = p.qkv_acc + (uint64_t)kvh * G * hd + (i / hd) * hd;
            qa[u] = src[d];
            qb[u] = src[rope_partner(d, p.half)];
            const uint32_t td = d < p.half ? d : (d < 2 * p.half ? d - p.half : 0u);
            qc[u] = rot ? ct[td] : 1.f;
            qsn[u] = rot ? st[td] : 0.f;
        }
        if (has_new && t < hd) {
            ka = p.qkv_acc[qd + head_off + t];
            kb = p.qkv_acc[qd + head_off + rope_partner(t, p.half)];
            va = p.qkv_acc[qd + kv_stride + head_off + t];
            const uint32_t td = t < p.half ? t : (t < 2 * p.half ? t - p.half : 0u);
            kc_ = rot ? ct[td] : 1.f;
            ks_ = rot ? st[td] : 0.f;
        }
    }
    // The q set-up's loads stay ahead of the cache rows, so a wait for them
    // does not also wait for the rows (loads complete in issue order). The
    // row loads are unconditional (a pass past the split re-reads its last
    // row; the address is clamped): loads under a branch would leave the
    // compiler's wait counts conservative, waiting for every load in flight.
    __builtin_amdgcn_sched_barrier(0);
    load_rows(kr, kc, p0 + (uint32_t)wave * PP);
    load_rows(vr, vcache, p0 + (uint32_t)wave * PP);
    __builtin_amdgcn_sched_barrier(0);

    // ---- q of the G heads (rotated, RMSNorm factor applied) and the appended row: threads 0..255 ----
    if (t < 256) {
        if (model) {
            const float inv = 1.0f / sqrtf(wave_sum(lane < p.ss_n ? ssp : 0.f) / (float)p.norm_n + 1e-6f);
            auto rot_val = [&](long long a_, long long b_, uint32_t d, float c, float sn) -> float {
                const float a = inv * from_fixed(a_);
                if (!rot || d >= 2 * p.half) return a;
                const float b = inv * from_fixed(b_);
                return d < p.half ? a * c - b * sn : a * c + b * sn;
            };
#pragma unroll
            for (uint32_t u = 0; u < QPT; ++u) {
                const uint32_t i = t + 256u * u;
                if (i < G * hd) qs[(i / hd) * HD + i % hd] = rot_val(qa[u], qb[u], i % hd, qc[u], qsn[u]);
            }
            if (has_new && t < hd) {
                float kv = rot_val(ka, kb, t, kc_, ks_);
                float vv = inv * from_fixed(va);
                const uint16_t kh = f2h(kv), vh = f2h(vv);
                const uint64_t idx = (uint64_t)cur * cps + coff + t;
                reinterpret_cast<uint16_t*>(p.kc)[idx] = kh;
                reinterpret_cast<uint16_t*>(p.vc)[idx] = vh;
                knew[t] = h2f(kh);                   // the stored values, as later steps read them
                vnew[t] = h2f(vh);
            }
        } else {
            for (uint32_t i = t; i < G * hd; i += 256)
                qs[(i / hd) * HD + i % hd] = p.q[(uint64_t)(kvh * G + i / hd) * hd + i % hd];
        }
    }
    __syncthreads();

    float qv[G4][VD];
#pragma unroll
    for (int g = 0; g < G4; ++g)
#pragma unroll
        for (int d = 0; d < VD; ++d) qv[g][d] = (uint32_t)g < G ? qs[g * HD + vc * VD + d] : 0.f;
    // scores in log2 units (scale * log2 e): the weights 2^(s - m) are e^(s' - m')
    // of the natural-log scores, one v_exp_f32 each; m goes out as m ln 2
    const float scale2 = p.scale * 1.4426950408889634f;
    float m[G4], l[G4], o[G4][VD];
#pragma unroll
    for (int g = 0; g < G4; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int d = 0; d < VD; ++d) o[g][d] = 0.f;
    }
    // Each wave's passes: wave, wave + NWV, ... Row i of the next pass goes
    // into the K registers as soon as row i's scores are done, and into the V
    // registers after row i's p.V, so one pass's loads overlap the other's
    // arithmetic.
    for (uint32_t pi = wave; pi < npass; pi += NWV) {
        const uint32_t c0 = p0 + pi * PP;
        const uint32_t cn = min((uint32_t)PP, p1 - c0);
        const uint32_t pn = pi + NWV;                  // this wave's next pass
        // ---- scores of the lane's positions: partial dots, summed over the row's 16 lanes ----
        float s[NI][G4];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t pos = c0 + 4u * i + vj;
            float k[VD];
            if constexpr (VD == 8) {
                const uint32_t w4[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    k[2 * e] = h2f((uint16_t)(w4[e] & 0xFFFFu));
                    k[2 * e + 1] = h2f((uint16_t)(w4[e] >> 16));
                }
            } else {
                const uint32_t w2[2] = {kr[i].x, kr[i].y};
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    k[2 * e] = h2f((uint16_t)(w2[e] & 0xFFFFu));
                    k[2 * e + 1] = h2f((uint16_t)(w2[e] >> 16));
                }
            }
            if (has_new && pos == cur) {
#pragma unroll
                for (int d = 0; d < VD; ++d) k[d] = knew[vc * VD + d];
            }
#pragma unroll
            for (int g = 0; g < G4; ++g) {
                float a = 0.f;
#pragma unroll
                for (int d = 0; d < VD; ++d) a = fmaf(qv[g][d], k[d], a);
                a = row16_sum(a);
                s[i][g] = 4u * i + vj < cn ? a * scale2 : -INFINITY;
            }
            load_row(kr[i], kc, p0 + pn * PP, i);     // row i of the next pass, as soon as it is free
        }
        // ---- online softmax per head over the pass ----
        float f[G4];
#pragma unroll
        for (int g = 0; g < G4; ++g) {
            float mx = s[0][g];
#pragma unroll
            for (int i = 1; i < NI; ++i) mx = fmaxf(mx, s[i][g]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            const float m_new = fmaxf(m[g], mx);
            // v_exp_f32 itself: arguments <= 0, and weights below 2^-126 (flushed
            // to zero) cannot reach a sum that holds the maximum's 1
            f[g] = __builtin_amdgcn_exp2f(m[g] - m_new);   // 0 on the first pass
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float e = 4u * i + vj < cn ? __builtin_amdgcn_exp2f(s[i][g] - m_new) : 0.f;
                s[i][g] = e;
                sum += e;
            }
            sum += __shfl_xor(sum, 16, kWave);
            sum += __shfl_xor(sum, 32, kWave);
            l[g] = l[g] * f[g] + sum;
            m[g] = m_new;
        }
        // ---- o[g] = o[g] f[g] + sum over the lane's positions of e V ----
#pragma unroll
        for (int g = 0; g < G4; ++g)
#pragma unroll
            for (int d = 0; d < VD; ++d) o[g][d] *= f[g];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (4u * i + vj < cn) {
            float v[VD];
            if constexpr (VD == 8) {
                const uint32_t w4[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] = h2f((uint16_t)(w4[e] & 0xFFFFu));
                    v[2 * e + 1] = h2f((uint16_t)(w4[e] >> 16));
                }
            } else {
                const uint32_t w2[2] = {vr[i].x, vr[i].y};
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    v[2 * e] = h2f((uint16_t)(w2[e] & 0xFFFFu));
                    v[2 * e + 1] = h2f((uint16_t)(w2[e] >> 16));
                }
            }
            if (has_new && c0 + 4u * i + vj == cur) {
#pragma unroll
                for (int d = 0; d < VD; ++d) v[d] = vnew[vc * VD + d];
            }
#pragma unroll
            for (int g = 0; g < G4; ++g)
#pragma unroll
                for (int d = 0; d < VD; ++d) o[g][d] = fmaf(s[i][g], v[d], o[g][d]);
            }
            load_row(vr[i], vcache, p0 + pn * PP, i);
        }
    }
    // ---- this wave's totals: sum the four position phases (lanes c, c + 16, c + 32, c + 48) ----
#pragma unroll
    for (int g = 0; g < G4; ++g)
#pragma unroll
        for (int d = 0; d < VD; ++d) {
            float v = o[g][d];
            v += __shfl_xor(v, 16, kWave);
            v += __shfl_xor(v, 32, kWave);
            o[g][d] = v;
        }
    if (vj == 0) {
#pragma unroll
        for (int g = 0; g < G4; ++g)
#pragma unroll
            for (int d = 0; d < VD; ++d) red_o[wave][g][vc * VD + d] = o[g][d];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G4; ++g) {
            red_m[wave][g] = m[g];
            red_l[wave][g] = l[g];
        }
    }
    __syncthreads();
    // ---- merge the waves in order: thread (g, d) ----
    if (t >= G * HD) return;
    const uint32_t g = t / HD, d = t % HD;
    float mx = -INFINITY;
    for (int w = 0; w < NWV; ++w) mx = fmaxf(mx, red_m[w][g]);
    float acc = 0.f, lt = 0.f;
    for (int w = 0; w < NWV; ++w) {
        const float wt = exp2f(red_m[w][g] - mx);  // 0 for a wave without passes
        acc = fmaf(red_o[w][g][d], wt, acc);
        lt = fmaf(red_l[w][g], wt, lt);
    }
    float* part = p.part + (((uint64_t)kvh * p.s_max + split) * G + g) * (hd + 2);
    part[d] = acc;
    if (d == 0) {
        part[hd] = mx * 0.6931471805599453f;       // natural-log units for the merge
        part[hd + 1] = lt;
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
    const uint32_t chunk = p.chunk ? p.chunk : attn_chunk_for(L);
    const uint32_t s_act = min(p.s_max, (L + chunk - 1) / chunk);
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
    kernarg_warm(p);
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
