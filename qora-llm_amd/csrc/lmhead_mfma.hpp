// Tied lm_head on the gfx950 integer matrix cores (v_mfma_i32_16x16x64_i8).
//
// logits[r] = sum_g s[r][g] * sum_{c in g} x[c] * (q[r][c] - 8)
//   (lm_head_parallel_q4, gemv.rs:825-864; groups of 32 along the hidden dim)
//
// Unlike the projection GEMVs, the scale here belongs to the output row, so
// the input vector alone is quantised: x[c] = M[c] * 2^(E-30) with 2^E
// bounding max |x| and M split into four signed base-256 limbs. One MFMA
// takes a 64-column block = two scale groups: A rows 0..3 hold the limbs of
// group 2p (columns 0..31 of the block, zeros elsewhere) and rows 4..7 those
// of group 2p+1 (columns 32..63), so
//   C[r][j]     = sum over group 2p   of limb_r * 16 (q - 8)   (lanes 0..15)
//   C[4 + r][j] = sum over group 2p+1 of limb_r * 16 (q - 8)   (lanes 16..31)
// for output row j. Each lane combines its four limb sums exactly in int32
// halves, converts once to fp32 and multiplies by its own group's scale.
// The group sums are exact; the fp32 steps after them round like the
// reference's own fp32 accumulation (the quantisation of x is 2^-30 of
// max |x|).
//
// Operand layouts (lane l, byte b = 0..15):
//   A[i = l % 16][k = 16 (l / 16) + b], B[k = 16 (l / 16) + b][j = l % 16],
//   C[i = 4 (l / 16) + r][j = l % 16] in result register r.
// Tile layout, 16 rows per tile (params.hpp, LmHeadParams): unit u of a
// tile is one 16-byte load per lane holding the B fragments of column
// blocks 2u and 2u+1 (8 bytes each; byte m of word w holds column
// 8w + m in its high nibble and 8w + 4 + m in its low nibble, the same
// order as the projection GEMV's fragments), and one 4-byte scale pair per
// lane l < 32: groups 4u + l/16 and 4u + 2 + l/16 of row l % 16.
#pragma once

#include "common.hpp"
#include "gemv_mfma.hpp"
#include "params.hpp"

namespace qora {

// One thread per (tile, unit, lane): the lane's 16-byte fragment pair and,
// for lanes 0..31, its scale pair. Rows past `rows` get q = 8 and scale 0.
__global__ __launch_bounds__(256) void lmhead_q4m_pack_kernel(const uint8_t* w, const uint16_t* scales, uint32_t rows,
                                                              uint32_t cols, uint32_t tiles, uint8_t* tw,
                                                              uint32_t* ts) {
    const uint32_t upt = cols / 128;
    const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (gid >= (uint64_t)tiles * upt * 64u) return;
    const uint32_t l = (uint32_t)(gid % 64u);
    const uint64_t tu = gid / 64u;
    const uint32_t u = (uint32_t)(tu % upt);
    const uint32_t tile = (uint32_t)(tu / upt);
    const uint32_t r = tile * 16u + l % 16u;
    const bool ok = r < rows;
    const uint8_t* row = w + (uint64_t)min(r, rows - 1u) * (cols / 2u);
    uint32_t word[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t c0 = 64u * (2u * u + (uint32_t)h) + 16u * (l / 16u);
#pragma unroll
        for (int wi = 0; wi < 2; ++wi) {
            uint32_t v = 0;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t ch = c0 + 8u * (uint32_t)wi + (uint32_t)m, cl = ch + 4u;
                const uint32_t qh = ok ? (row[ch / 2u] >> ((ch & 1u) * 4u)) & 0xFu : 8u;
                const uint32_t ql = ok ? (row[cl / 2u] >> ((cl & 1u) * 4u)) & 0xFu : 8u;
                v |= ((qh << 4) | ql) << (8 * m);
            }
            word[2 * h + wi] = v;
        }
    }
    *reinterpret_cast<uint4*>(tw + gid * 16u) = make_uint4(word[0], word[1], word[2], word[3]);
    if (l < 32u) {
        const uint64_t G = cols / 32u;
        const uint32_t g0 = 4u * u + l / 16u;
        const uint32_t s0 = ok ? scales[(uint64_t)r * G + g0] : 0u;
        const uint32_t s1 = ok ? scales[(uint64_t)r * G + g0 + 2u] : 0u;
        ts[tu * 32u + l] = s0 | (s1 << 16);
    }
}

// exact sum of a lane's four limb sums as fp32: (C0 + 2^8 C1) + 2^16 (C2 + 2^8 C3)
__device__ __forceinline__ float lm_limb_value(v4i32 c) {
    const int lo = c[0] + (c[1] << 8);
    const int hi = c[2] + (c[3] << 8);
    return fmaf((float)hi, 65536.0f, (float)lo);
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < NT / kWave; ++i) m = fmaxf(m, red[i]);
    return m;
}

// Four waves; wave w of block b takes tiles gw, gw + W, gw + 2W, ... (gw =
// 4b + w, W = 4 * gridDim.x). Each wave keeps one whole tile of loads in
// flight: unit u of the next tile is loaded into the registers of unit u of
// the current one as soon as they are consumed. The input loads are issued
// before the first tile's, so waiting for x does not wait for weights.
// FIXED: the input is the fixed-point residual p.xacc with the RMSNorm
// prologue (gamma p.gamma); otherwise the fp32 vector p.x as is.
template <int NP, bool FIXED>
__global__ __launch_bounds__(256) void lmhead_q4m_kernel(LmHeadParams p) {
    kernarg_warm(p);
    constexpr int NT = 256, NW = 4;
    constexpr int UPT = NP / 2;                 // 16-byte units per lane per tile
    constexpr int COLS = 64 * NP;
    constexpr int XPT = (COLS + NT - 1) / NT;   // inputs per thread
    constexpr int SLOT = 272;                   // LDS bytes per column block: 16 A slots + a zero slot
    static_assert(NP % 2 == 0 && NP >= 2 && NP <= 32, "cols = 128 .. 2048");
    __shared__ __align__(16) uint8_t xl[NP * SLOT];
    __shared__ float red[NW];
    __shared__ float s_val[NW];
    __shared__ uint32_t s_idx[NW];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const uint32_t W = gridDim.x * NW;
    const uint32_t last = p.tiles - 1u;
    uint32_t tile = blockIdx.x * NW + (uint32_t)wave;

    // ---- inputs ----
    long long xa[FIXED ? XPT : 1];
    float xf[FIXED ? 1 : XPT];
    uint16_t gm[FIXED ? XPT : 1];
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const uint32_t c = min((uint32_t)(t + NT * j), (uint32_t)COLS - 1u);
        if constexpr (FIXED) {
            xa[j] = p.xacc[c];
            gm[j] = p.gamma[c];
        } else {
            xf[j] = p.x[c];
        }
    }

    // ---- first tile (clamped: a wave with no tile loads the last one and skips it) ----
    uint4 wb[UPT];
    uint32_t sb[UPT];
    {
        const uint32_t tl = min(tile, last);
        const uint8_t* wp = p.tw + (uint64_t)tl * UPT * 1024u + (uint32_t)lane * 16u;
        const uint32_t* sp = p.ts + (uint64_t)tl * UPT * 32u + ((uint32_t)lane & 31u);
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            wb[u] = ld_stream(wp + u * 1024);
            sb[u] = ld_stream1(sp + u * 32);
        }
    }

    // ---- RMSNorm (optional), block exponent, limb bytes into LDS ----
    float xv[XPT];
    float ss = 0.f, mx = 0.f;
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const bool ok = t + NT * j < COLS;
        float v = 0.f;
        if constexpr (FIXED) {
            v = ok ? from_fixed(xa[j]) : 0.f;
            fix_flag(p.range_flag, ok && fix_out_of_range(xa[j], kFixReadLimit));
        } else {
            v = ok ? xf[j] : 0.f;
        }
        xv[j] = v;
        ss += v * v;
    }
    if constexpr (FIXED) {
        ss = block_sum<NT>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)COLS + 1e-6f);
#pragma unroll
        for (int j = 0; j < XPT; ++j) xv[j] = xv[j] * inv * h2f(gm[j]);
    }
#pragma unroll
    for (int j = 0; j < XPT; ++j) mx = fmaxf(mx, fabsf(xv[j]));
    mx = block_max<NT>(mx, red);
    const int ex = mx > 0.f ? (int)((__float_as_uint(mx) >> 23) & 0xFFu) - 126 : 0;
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const uint32_t c = (uint32_t)(t + NT * j);
        if (c < (uint32_t)COLS) {
            const int M = (int)rintf(ldexpf(xv[j], 30 - ex));
            const uint32_t limbs = (uint32_t)(M + 0x808080) ^ 0x808080u;
            uint8_t* dst = xl + (c / 64u) * SLOT + ((c % 64u) / 16u) * 64u + (c % 16u);
            dst[0] = (uint8_t)(limbs & 0xFFu);
            dst[16] = (uint8_t)((limbs >> 8) & 0xFFu);
            dst[32] = (uint8_t)((limbs >> 16) & 0xFFu);
            dst[48] = (uint8_t)(limbs >> 24);
        }
    }
    for (int i = t; i < NP * 4; i += NT) *reinterpret_cast<uint32_t*>(xl + (i / 4) * SLOT + 256 + (i % 4) * 4) = 0u;
    __syncthreads();

    // A operand: rows 0..3 carry group 2p (lanes with l/16 < 2), rows 4..7
    // group 2p+1 (l/16 >= 2); every other lane reads the zero slot.
    const uint32_t li = (uint32_t)lane % 16u, kq = (uint32_t)lane / 16u;
    const bool nz = li < 8u && (li >> 2) == (kq >> 1);
    const uint32_t aoff = nz ? kq * 64u + (li & 3u) * 16u : 256u;
    const v4i32 zero = (v4i32){0, 0, 0, 0};

    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    for (; tile < p.tiles; tile += W) {
        // re-read the A fragments from LDS every tile rather than holding all
        // of them in registers, which would halve the waves per SIMD
        uint32_t ao = aoff;
        asm volatile("" : "+v"(ao));
        const uint32_t nx = min(tile + W, last);
        const uint8_t* wp = p.tw + (uint64_t)nx * UPT * 1024u + (uint32_t)lane * 16u;
        const uint32_t* sp = p.ts + (uint64_t)nx * UPT * 32u + ((uint32_t)lane & 31u);
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            const uint4 w = wb[u];
            const uint32_t s2 = sb[u];
            wb[u] = ld_stream(wp + u * 1024);
            sb[u] = ld_stream1(sp + u * 32);
            const v4i32 a0 = *reinterpret_cast<const v4i32*>(xl + (2 * u) * SLOT + ao);
            const v4i32 a1 = *reinterpret_cast<const v4i32*>(xl + (2 * u + 1) * SLOT + ao);
            const v4i32 c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, q4_bfrag(w.x, w.y), zero, 0, 0, 0);
            const v4i32 c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, q4_bfrag(w.z, w.w), zero, 0, 0, 0);
            acc = fmaf(lm_limb_value(c0), f16lo(s2), acc);
            acc = fmaf(lm_limb_value(c1), f16hi(s2), acc);
        }
        // lanes 0..15 hold the even groups of row l, lanes 16..31 the odd ones
        acc += __shfl_xor(acc, 16, kWave);
        const float y = ldexpf(acc, ex - 34);
        const uint32_t r = tile * 16u + (uint32_t)lane;
        if (lane < 16 && r < p.rows) {
            p.y[r] = y;
            if (argmax_better(y, r, best_v, best_i)) {
                best_v = y;
                best_i = r;
            }
        }
    }

    if (!p.do_argmax) return;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best_v, off, kWave);
        const uint32_t oi = __shfl_xor(best_i, off, kWave);
        if (argmax_better(ov, oi, best_v, best_i)) {
            best_v = ov;
            best_i = oi;
        }
    }
    if (lane == 0) {
        s_val[wave] = best_v;
        s_idx[wave] = best_i;
    }
    __syncthreads();
    if (t == 0) {
        float bv = s_val[0];
        uint32_t bi = s_idx[0];
        for (int w = 1; w < NW; ++w)
            if (argmax_better(s_val[w], s_idx[w], bv, bi)) {
                bv = s_val[w];
                bi = s_idx[w];
            }
        p.part_val[blockIdx.x] = bv;
        p.part_idx[blockIdx.x] = bi;
    }
}

}  // namespace qora
