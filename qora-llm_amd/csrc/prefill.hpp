// Batched prefill (raw_prefill, gemv.rs:1027-1190): the prompt's tokens go
// through every layer together, so each weight is streamed once per block of
// 64 tokens instead of once per token, and the projections run on the gfx950
// matrix cores (v_mfma_f32_16x16x32_f16).
//
// Numerics of the GEMM (gemm_q4 / gemm_f16, gemv.rs:569-588, 677-706):
//   y[t][n] = sum_k x[t][k] * w[k][n], w = s[k][n/32] * (q - 8) (Q4) or the f16
//   value. Both operands are split into two binary16 parts on a power-of-two
//   scale, so no product loses more than fp32 would:
//     x' = x * 2^-e_t     (e_t per token row, |x'| < 2^15),  x' = xh + xl
//     w' = w * 2^-f_g     (f_g per 32-column group, |w'| <= 2^15), w' = wh + wl
//   with xh = f16(x'), xl = f16(x' - xh) (22 significant bits of x') and, for
//   Q4, wh + wl == w' exactly (s has 11 significant bits, q - 8 at most 3).
//   acc = xh wh + xh wl + xl wh summed in fp32 by the matrix cores (each
//   f16 x f16 product is exact in fp32; the dropped xl wl is below 2^-22 of the
//   product), and y = acc * 2^(e_t + f_g) exactly. F16 weights have wl = 0.
//   So the result is fp32 accumulation of (nearly) exact products: it differs
//   from the reference only in summation order and in the last bits of x.
//
// The GEMM block is 256 threads (2 x 2 waves) over 64 tokens x NT columns;
// each step stages a 32-deep K slice of x' (both parts, from the split
// buffers) and of w' (dequantised from the reference-layout weights) in LDS,
// double-buffered, with the next slice's global loads in flight during the
// current slice's MFMAs.
//
// Operand layouts of v_mfma_f32_16x16x32_f16 (lane l, element b = 0..7):
//   A[i = l % 16][k = 8 (l / 16) + b], B[k = 8 (l / 16) + b][j = l % 16],
//   C[i = 4 (l / 16) + r][j = l % 16] in result register r.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace qora {

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

// Power-of-two exponent e with |v| * 2^-e < 2^15 for every |v| <= amax.
__device__ __forceinline__ int pf_row_exponent(float amax) {
    int E = 0;
    (void)frexpf(amax, &E);      // amax < 2^E (E = 0 for amax = 0)
    return E - 15;
}

__device__ __forceinline__ void pf_split(float v, int e, _Float16* hi, _Float16* lo) {
    const float s = ldexpf(v, -e);
    const _Float16 h = (_Float16)s;
    *hi = h;
    *lo = (_Float16)(s - (float)h);
}

template <int NT>
__device__ __forceinline__ float pf_block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < NT / kWave; ++w) m = fmaxf(m, red[w]);
    return m;
}

// ---------------------------------------------------------------------------
// Row producers: one block of 256 threads per token row. Each writes the
// split GEMM operand (xh, xl: [T][k] binary16, xe[T] exponents).
// ---------------------------------------------------------------------------

// Embedding rows (embed_lookup, gemv.rs:515-526, 710-736): x[t] = dequant(E[ids[t]]).
__global__ __launch_bounds__(256) void pf_embed_kernel(PrefillRowParams p) {
    const uint32_t t = blockIdx.x;
    const uint32_t tok = min(p.ids[t], p.vocab - 1u);
    float* x = p.x + (uint64_t)t * p.n;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) {
        float v;
        if (p.fmt == FMT_Q4) {
            const uint64_t G = p.n / 32;
            const uint8_t b = p.emb_w[(uint64_t)tok * G * 16 + j / 2];
            const int q = (j & 1) ? (b >> 4) : (b & 0x0F);
            v = h2f(p.emb_s[(uint64_t)tok * G + j / 32]) * (float)(q - 8);
        } else {
            v = h2f(reinterpret_cast<const uint16_t*>(p.emb_w)[(uint64_t)tok * p.n + j]);
        }
        x[j] = v;
    }
}

// RMSNorm (rms_norm_f16, gemv.rs:744-753): v = (x * inv) * gamma, then split.
__global__ __launch_bounds__(256) void pf_rmsnorm_split_kernel(PrefillRowParams p) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    const float* x = p.x + (uint64_t)t * p.n;
    float ss = 0.f;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) ss = fmaf(x[j], x[j], ss);
    ss = block_sum<256>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)p.n + 1e-6f);
    float amax = 0.f;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) amax = fmaxf(amax, fabsf((x[j] * inv) * h2f(p.gamma[j])));
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) pf_split((x[j] * inv) * h2f(p.gamma[j]), e, xh + j, xl + j);
    if (threadIdx.x == 0) p.xe[t] = e;
}

// Plain split of an fp32 row (the attention output, input of the o projection).
__global__ __launch_bounds__(256) void pf_split_kernel(PrefillRowParams p) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    const float* x = p.x + (uint64_t)t * p.n;
    float amax = 0.f;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) amax = fmaxf(amax, fabsf(x[j]));
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) pf_split(x[j], e, xh + j, xl + j);
    if (threadIdx.x == 0) p.xe[t] = e;
}

// SwiGLU (gemv.rs:1160-1166): v = (g / (1 + exp(-g))) * u over the gate and up
// rows, then split (the down projection's input).
__global__ __launch_bounds__(256) void pf_silu_split_kernel(PrefillRowParams p) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    const float* g = p.x + (uint64_t)t * p.ld;
    const float* u = p.u + (uint64_t)t * p.ld;
    float amax = 0.f;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) {
        const float gv = g[j];
        amax = fmaxf(amax, fabsf((gv / (1.0f + expf(-gv))) * u[j]));
    }
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) {
        const float gv = g[j];
        pf_split((gv / (1.0f + expf(-gv))) * u[j], e, xh + j, xl + j);
    }
    if (threadIdx.x == 0) p.xe[t] = e;
}

// ---------------------------------------------------------------------------
// Per-group weight exponents f_g (Q4): |s[k][g] * (q - 8)| <= 2^(eb + 3) with
// |s| <= 2^eb over the column group, so f_g = eb - 12 keeps |w'| <= 2^15.
// One thread per group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pf_weight_exp_kernel(const uint16_t* scales, uint32_t k, uint32_t groups,
                                                            int8_t* wf) {
    const uint32_t g = blockIdx.x * 256u + threadIdx.x;
    if (g >= groups) return;
    uint32_t mx = 0;
    for (uint32_t r = 0; r < k; ++r) mx = max(mx, (uint32_t)(scales[(uint64_t)r * groups + g] & 0x7FFFu));
    const int e = (int)((mx >> 10) & 0x1F);
    const int eb = e == 0 ? -14 : e - 14;      // |s| <= 2^eb (infinities and NaN: e = 31)
    wf[g] = (int8_t)(eb - 12);
}

// ---------------------------------------------------------------------------
// The GEMM. Grid (n / NT column tiles, ceil(T / 64) token tiles).
// ---------------------------------------------------------------------------
template <int NT, bool Q4>
__global__ __launch_bounds__(256) void pf_gemm_kernel(PrefillGemmParams p) {
    constexpr int MT = 64, KC = 32;
    constexpr int XS = KC + 8;                      // LDS row stride in halves (80 B: 16-B aligned, no read conflicts)
    constexpr int WN = NT / 2;                      // columns per wave
    constexpr int TN = WN / 16;                     // 16-column MFMA tiles per wave
    constexpr int RPT = NT / 16;                    // weight rows per thread per slice (8 or 4)
    __shared__ __align__(16) _Float16 xs[2][2][MT * XS];
    __shared__ __align__(16) _Float16 ws[2][Q4 ? 2 : 1][NT * XS];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t n0 = blockIdx.x * NT;
    const uint32_t m0 = blockIdx.y * MT;
    const uint32_t K = p.k, N = p.n;
    const uint32_t groups = N / 32;

    // x' slice: thread t loads 16 B of row t / 4 (hi and lo)
    const uint32_t xr = (uint32_t)t >> 2, xp = (uint32_t)t & 3u;
    const bool xrow_ok = m0 + xr < p.T;
    const uint64_t xoff = (uint64_t)(m0 + (xrow_ok ? xr : 0u)) * K + xp * 8u;
    // w' slice: thread t takes columns 2 bc, 2 bc + 1 of rows RPT rg .. RPT rg + RPT - 1
    const uint32_t bc = (uint32_t)t % (NT / 2), rg = (uint32_t)t / (NT / 2);
    const uint32_t col = n0 + 2u * bc;
    const uint32_t colc = min(col, N - 2u);         // clamped (masked tail of the last tile)
    const uint32_t grp = colc / 32u;
    float wscale = 1.0f;                            // 2^-f_g
    if constexpr (Q4) wscale = ldexpf(1.0f, -(int)p.wf[grp]);

    uint4 xh_r, xl_r;
    uint32_t wq[RPT];                               // Q4: byte (2 columns) per row; F16: 2 halves per row
    uint16_t sc[Q4 ? RPT : 1];

    auto load_slice = [&](uint32_t k0) {
        if (xrow_ok) {
            xh_r = *reinterpret_cast<const uint4*>(p.xh + xoff + k0);
            xl_r = *reinterpret_cast<const uint4*>(p.xl + xoff + k0);
        } else {
            xh_r = make_uint4(0, 0, 0, 0);
            xl_r = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const uint64_t row = k0 + rg * RPT + r;
            if constexpr (Q4) {
                wq[r] = p.w[row * (N / 2) + colc / 2];
                sc[r] = p.scales[row * groups + grp];
            } else {
                wq[r] = *reinterpret_cast<const uint32_t*>(p.w + (row * N + colc) * 2);
            }
        }
    };

    auto store_slice = [&](int buf) {
        *reinterpret_cast<uint4*>(&xs[buf][0][xr * XS + xp * 8]) = xh_r;
        *reinterpret_cast<uint4*>(&xs[buf][1][xr * XS + xp * 8]) = xl_r;
        // two columns, RPT consecutive k each
        _Float16 h0[RPT], h1[RPT], l0[RPT], l1[RPT];
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            if constexpr (Q4) {
                const float s = h2f(sc[r]) * wscale;            // exact: power-of-two scaling
                const float w0 = s * (float)((int)(wq[r] & 0xFu) - 8);
                const float w1 = s * (float)((int)(wq[r] >> 4) - 8);
                h0[r] = (_Float16)w0;
                h1[r] = (_Float16)w1;
                l0[r] = (_Float16)(w0 - (float)h0[r]);
                l1[r] = (_Float16)(w1 - (float)h1[r]);
            } else {
                h0[r] = __builtin_bit_cast(_Float16, (uint16_t)(wq[r] & 0xFFFFu));
                h1[r] = __builtin_bit_cast(_Float16, (uint16_t)(wq[r] >> 16));
            }
        }
        _Float16* c0h = &ws[buf][0][(2u * bc) * XS + rg * RPT];
        _Float16* c1h = &ws[buf][0][(2u * bc + 1u) * XS + rg * RPT];
        if constexpr (RPT == 8) {
            *reinterpret_cast<half8v*>(c0h) = half8v{h0[0], h0[1], h0[2], h0[3], h0[4], h0[5], h0[6], h0[7]};
            *reinterpret_cast<half8v*>(c1h) = half8v{h1[0], h1[1], h1[2], h1[3], h1[4], h1[5], h1[6], h1[7]};
        } else {
#pragma unroll
            for (int r = 0; r < RPT; ++r) { c0h[r] = h0[r]; c1h[r] = h1[r]; }
        }
        if constexpr (Q4) {
            _Float16* c0l = &ws[buf][1][(2u * bc) * XS + rg * RPT];
            _Float16* c1l = &ws[buf][1][(2u * bc + 1u) * XS + rg * RPT];
            if constexpr (RPT == 8) {
                *reinterpret_cast<half8v*>(c0l) = half8v{l0[0], l0[1], l0[2], l0[3], l0[4], l0[5], l0[6], l0[7]};
                *reinterpret_cast<half8v*>(c1l) = half8v{l1[0], l1[1], l1[2], l1[3], l1[4], l1[5], l1[6], l1[7]};
            } else {
#pragma unroll
                for (int r = 0; r < RPT; ++r) { c0l[r] = l0[r]; c1l[r] = l1[r]; }
            }
        }
    };

    f32x4v acc[2][TN];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    const uint32_t li = (uint32_t)lane % 16u, kq = (uint32_t)lane / 16u;
    const uint32_t steps = K / KC;
    load_slice(0);
    store_slice(0);
    __syncthreads();
    for (uint32_t s = 0; s < steps; ++s) {
        const int buf = (int)(s & 1u);
        if (s + 1 < steps) load_slice((s + 1) * KC);
        half8v ah[2], al[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t row = (uint32_t)wm * 32u + (uint32_t)i * 16u + li;
            ah[i] = *reinterpret_cast<const half8v*>(&xs[buf][0][row * XS + kq * 8u]);
            al[i] = *reinterpret_cast<const half8v*>(&xs[buf][1][row * XS + kq * 8u]);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t c = (uint32_t)wn * WN + (uint32_t)j * 16u + li;
            const half8v bh = *reinterpret_cast<const half8v*>(&ws[buf][0][c * XS + kq * 8u]);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh, acc[i][j], 0, 0, 0);
            }
            if constexpr (Q4) {
                const half8v bl = *reinterpret_cast<const half8v*>(&ws[buf][1][c * XS + kq * 8u]);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl, acc[i][j], 0, 0, 0);
            }
        }
        if (s + 1 < steps) store_slice(buf ^ 1);
        __syncthreads();
    }

    // epilogue: y = acc * 2^(e_t + f_g), stored or added to the residual rows
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t c = n0 + (uint32_t)wn * WN + (uint32_t)j * 16u + li;
            if (c >= N) continue;
            const int fg = Q4 ? (int)p.wf[c / 32u] : 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t row = m0 + (uint32_t)wm * 32u + (uint32_t)i * 16u + kq * 4u + (uint32_t)r;
                if (row >= p.T) continue;
                const float v = ldexpf(acc[i][j][r], p.xe[row] + fg);
                float* y = p.y + (uint64_t)row * p.ldy + c;
                if (p.accumulate) *y += v;
                else *y = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// RoPE and cache append (gemv.rs:1062-1083): q|k|v rows of tokens pos0 + t.
// q (rotated) goes to q_out [T][H][hd]; k (rotated) and v to the cache rows.
// One block per token.
// ---------------------------------------------------------------------------
template <bool F16KV>
__global__ __launch_bounds__(256) void pf_rope_cache_kernel(PrefillAttnParams p) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = p.pos0 + t;
    const uint32_t hd = p.hd, half = p.half;
    const uint32_t qd = p.H * hd, kvd = p.KVH * hd;
    const float* row = p.qkv + (uint64_t)t * (qd + 2 * kvd);
    const float* ct = p.rope_cos + (uint64_t)pos * half;
    const float* st = p.rope_sin + (uint64_t)pos * half;
    const bool rot = p.use_rope != 0;
    auto rotate = [&](const float* v, uint32_t i) -> float {
        const uint32_t d = i % hd, base = i - d;
        if (!rot || d >= 2 * half) return v[i];
        const float c = ct[d % half], s = st[d % half];
        // apply_rope_raw (gemv.rs:757-778): (x1, x2) -> (x1 c - x2 s, x2 c + x1 s)
        return d < half ? v[i] * c - v[base + d + half] * s : v[i] * c + v[base + d - half] * s;
    };
    for (uint32_t i = threadIdx.x; i < qd; i += 256) p.q[(uint64_t)t * qd + i] = rotate(row, i);
    const uint64_t crow = (uint64_t)pos * kvd;
    for (uint32_t i = threadIdx.x; i < kvd; i += 256) {
        const float kv = rotate(row + qd, i), vv = row[qd + kvd + i];
        if constexpr (F16KV) {
            reinterpret_cast<uint16_t*>(p.kc)[crow + i] = f2h(kv);
            reinterpret_cast<uint16_t*>(p.vc)[crow + i] = f2h(vv);
        } else {
            reinterpret_cast<float*>(p.kc)[crow + i] = kv;
            reinterpret_cast<float*>(p.vc)[crow + i] = vv;
        }
    }
}

// ---------------------------------------------------------------------------
// Causal attention of the chunk's tokens (gemv.rs:1088-1130): token pos0 + t,
// head h attends to cache positions [0, pos0 + t] of KV head h / groups, with
// scores dot(q, k) / sqrt(hd) and softmax over them. Block (32-token query
// tile, head): 32 queries x 32 keys per step from LDS, online softmax, 8
// threads per query row (4 keys and hd/8 output dims each). The cache values
// read back are the stored ones (binary16 for an f16 cache), as decode reads
// them.
// ---------------------------------------------------------------------------
template <bool F16KV>
__global__ __launch_bounds__(256) void pf_attn_kernel(PrefillAttnParams p) {
    constexpr int QT = 32, KT = 32, HDM = kAttnMaxHd;
    constexpr int KSTR = HDM + 4;
    __shared__ __align__(16) float qs[QT * HDM];
    __shared__ __align__(16) float ks[KT * KSTR];
    __shared__ __align__(16) float vs[KT * HDM];
    __shared__ float ps[QT * (KT + 1)];
    const uint32_t t = threadIdx.x;
    const uint32_t qt0 = blockIdx.x * QT;           // first query (chunk-relative)
    const uint32_t h = blockIdx.y;
    const uint32_t hd = p.hd, G = p.H / p.KVH, kvh = h / G;
    const uint32_t qd = p.H * hd, kvd = p.KVH * hd;
    const uint32_t nq = min((uint32_t)QT, p.T - qt0);
    const uint32_t qr = t / 8u, sub = t % 8u;       // query row, lane within the row's 8 threads
    const uint32_t qpos = p.pos0 + qt0 + qr;        // absolute position of this thread's query
    const bool qok = qr < nq;
    const uint32_t last = p.pos0 + qt0 + nq - 1u;   // last key position any query here needs
    const uint32_t dpt = hd / 8u;                   // output dims per thread (<= 16)

    for (uint32_t e = t; e < QT * hd; e += 256) {
        const uint32_t r = e / hd, d = e % hd;
        qs[r * HDM + d] = r < nq ? p.q[(uint64_t)(qt0 + r) * qd + (uint64_t)h * hd + d] : 0.f;
    }
    float m = -INFINITY, l = 0.f;
    float o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.f;

    for (uint32_t k0 = 0; k0 <= last; k0 += KT) {
        __syncthreads();                            // previous tiles consumed (and qs written)
        for (uint32_t e = t; e < KT * hd; e += 256) {
            const uint32_t r = e / hd, d = e % hd;
            const uint32_t kp = min(k0 + r, last);
            const uint64_t idx = (uint64_t)kp * kvd + (uint64_t)kvh * hd + d;
            float kv, vv;
            if constexpr (F16KV) {
                kv = h2f(reinterpret_cast<const uint16_t*>(p.kc)[idx]);
                vv = h2f(reinterpret_cast<const uint16_t*>(p.vc)[idx]);
            } else {
                kv = reinterpret_cast<const float*>(p.kc)[idx];
                vv = reinterpret_cast<const float*>(p.vc)[idx];
            }
            ks[r * KSTR + d] = kv;
            vs[r * HDM + d] = vv;
        }
        __syncthreads();
        // scores of keys sub, sub + 8, sub + 16, sub + 24
        float sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t kr = sub + 8u * (uint32_t)j;
            float a = 0.f;
            for (uint32_t d = 0; d < hd; d += 4) {
                const float4 qv = *reinterpret_cast<const float4*>(&qs[qr * HDM + d]);
                const float4 kv = *reinterpret_cast<const float4*>(&ks[kr * KSTR + d]);
                a = fmaf(qv.x, kv.x, a);
                a = fmaf(qv.y, kv.y, a);
                a = fmaf(qv.z, kv.z, a);
                a = fmaf(qv.w, kv.w, a);
            }
            sc[j] = (qok && k0 + kr <= qpos) ? a * p.scale : -INFINITY;
        }
        float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 2, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 4, kWave));
        const float m_new = fmaxf(m, mx);
        // a row whose keys are all masked keeps m = -inf: use 0 as the reference
        const float mref = m_new == -INFINITY ? 0.f : m_new;
        const float f = expf(m - mref);
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float e = expf(sc[j] - mref);       // 0 for masked keys
            ps[qr * (KT + 1) + sub + 8u * (uint32_t)j] = e;
            sum += e;
        }
        sum += __shfl_xor(sum, 1, kWave);
        sum += __shfl_xor(sum, 2, kWave);
        sum += __shfl_xor(sum, 4, kWave);
        l = l * f + sum;
        m = m_new;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] *= f;
        for (uint32_t kr = 0; kr < KT; ++kr) {
            const float pv = ps[qr * (KT + 1) + kr];
            const float* vr = &vs[kr * HDM + sub * dpt];
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if ((uint32_t)i < dpt) o[i] = fmaf(pv, vr[i], o[i]);
        }
    }
    if (!qok) return;
    const float inv = 1.0f / l;
    float* out = p.out + (uint64_t)(qt0 + qr) * qd + (uint64_t)h * hd + sub * dpt;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if ((uint32_t)i < dpt) out[i] = o[i] * inv;
}

}  // namespace qora
