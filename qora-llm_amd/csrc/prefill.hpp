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
// Two GEMM kernels share these numerics:
//   * pf_gemm2_kernel (every Q4 projection whose width is a multiple of
//     128): weights pre-packed once at set-up, 4 waves over BM tokens x 128
//     columns, only x' in LDS, each wave dequantising its own weights in
//     registers (its comment below has the details);
//   * pf_gemm_kernel (F16 weights and other widths): the reference layout
//     read directly, 2 x 2 waves over 64 tokens x NT columns, each 32-deep K
//     slice of x' and w' (dequantised) staged in LDS.
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

// Row chunks of the register-cached producers: thread t of NT owns the runs
// of four consecutive elements starting at 4 (t + NT i). A row whose length,
// stride and pointers are multiples of four elements (16 bytes of fp32, 8 of
// binary16) moves as vectors (VEC); any other row element by element, with
// the same values. Elements past the row end read as 0 and are not written.
// Loads are branch-free (indexes clamped into the row, the value then
// selected), so all of a thread's loads are in flight together.
__device__ __forceinline__ bool pf_al(const void* a, uintptr_t m) { return ((uintptr_t)a & (m - 1)) == 0; }

template <bool VEC>
__device__ __forceinline__ void pf_load4(const float* x, uint32_t j, uint32_t n, float* v) {
    if constexpr (VEC) {                            // n is a positive multiple of 4
        const float4 a = *reinterpret_cast<const float4*>(x + min(j, n - 4u));
        const bool in = j < n;
        v[0] = in ? a.x : 0.f;
        v[1] = in ? a.y : 0.f;
        v[2] = in ? a.z : 0.f;
        v[3] = in ? a.w : 0.f;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float a = x[min(j + (uint32_t)c, n - 1u)];
            v[c] = j + c < n ? a : 0.f;
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void pf_gamma4(const uint16_t* g, uint32_t j, uint32_t n, float* v) {
    if constexpr (VEC) {
        const uint2 a = *reinterpret_cast<const uint2*>(g + min(j, n - 4u));
        const bool in = j < n;
        v[0] = in ? h2f((uint16_t)(a.x & 0xFFFFu)) : 0.f;
        v[1] = in ? h2f((uint16_t)(a.x >> 16)) : 0.f;
        v[2] = in ? h2f((uint16_t)(a.y & 0xFFFFu)) : 0.f;
        v[3] = in ? h2f((uint16_t)(a.y >> 16)) : 0.f;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float a = h2f(g[min(j + (uint32_t)c, n - 1u)]);
            v[c] = j + c < n ? a : 0.f;
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void pf_store4(float* x, uint32_t j, uint32_t n, const float* v) {
    if constexpr (VEC) {
        if (j < n) *reinterpret_cast<float4*>(x + j) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (j + c < n) x[j + c] = v[c];
    }
}

template <bool VEC>
__device__ __forceinline__ void pf_split4(const float* v, int e, _Float16* xh, _Float16* xl, uint32_t j, uint32_t n) {
    typedef _Float16 half4v __attribute__((ext_vector_type(4)));
    if constexpr (VEC) {
        if (j >= n) return;
        half4v h, l;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float sv = ldexpf(v[c], -e);
            h[c] = (_Float16)sv;
            l[c] = (_Float16)(sv - (float)h[c]);
        }
        *reinterpret_cast<half4v*>(xh + j) = h;
        *reinterpret_cast<half4v*>(xl + j) = l;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (j + c < n) pf_split(v[c], e, xh + j + c, xl + j + c);
    }
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
    float* x = p.x + (uint64_t)t * p.n;
    if (p.part) {
        // split-K partials of the preceding residual add, summed in split order
        const float* pr = p.part + (uint64_t)t * p.n;
        for (uint32_t j = threadIdx.x; j < p.n; j += 256) {
            float a = pr[j];
            for (uint32_t z = 1; z < p.splits; ++z) a += pr[(uint64_t)z * p.part_stride + j];
            x[j] += a;
        }
        __syncthreads();
    }
    // sum of squares in the order of the register-cached kernel: thread t
    // takes the runs 4 t + 1024 i, each in element order
    float ss = 0.f;
    for (uint32_t b0 = 4u * threadIdx.x; b0 < p.n; b0 += 1024u)
        for (uint32_t j = b0; j < min(b0 + 4u, p.n); ++j) ss = fmaf(x[j], x[j], ss);
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
// p.u null: the rows already hold SiLU(g) * u (the gate|up GEMM's SwiGLU
// pairing), only split.
__global__ __launch_bounds__(256) void pf_silu_split_kernel(PrefillRowParams p) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    const bool swiglu = p.u != nullptr;
    const float* g = p.x + (uint64_t)t * p.ld;
    const float* u = swiglu ? p.u + (uint64_t)t * p.ld : g;
    auto h = [&](uint32_t j) {
        const float gv = g[j];
        return swiglu ? (gv / (1.0f + expf(-gv))) * u[j] : gv;
    };
    float amax = 0.f;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) amax = fmaxf(amax, fabsf(h(j)));
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
    for (uint32_t j = threadIdx.x; j < p.n; j += 256) pf_split(h(j), e, xh + j, xl + j);
    if (threadIdx.x == 0) p.xe[t] = e;
}

// The same three producers with the row held in registers: each element is
// read once instead of two or three times, with the same arithmetic. The
// norm and the split keep the runs of four elements at 4 (t + 256 i) (as
// pf_load4 describes; the norm's sum of squares runs in that order in the
// multi-pass kernel too). For rows of at most 256 * EPT (SwiGLU: NT * EPT).
template <int EPT, bool VEC>
__device__ __forceinline__ void pf_rmsnorm_split_row(const PrefillRowParams& p, float* red) {
    constexpr int C = EPT / 4;
    const uint32_t t = blockIdx.x;
    float* x = p.x + (uint64_t)t * p.n;
    float v[C][4];
    float gm[C][4];
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const uint32_t j = 4u * (threadIdx.x + 256u * (uint32_t)i);
        pf_load4<VEC>(x, j, p.n, v[i]);
        pf_gamma4<VEC>(p.gamma, j, p.n, gm[i]);
    }
    if (p.part) {
        // the residual add of the split-K GEMM before this norm, in the
        // order pf_splitk_reduce2_kernel sums: x += ((p0 + p1) + p2) + ...
        // Partials are loaded four splits at a time, all of a group's loads
        // issued before its adds (split indexes clamped to the last split;
        // the extra values are not added).
        const float* pr = p.part + (uint64_t)t * p.n;
        float a[C][4];
        for (uint32_t z = 0; z < p.splits; z += 4) {
            float q[4][C][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint64_t zo = (uint64_t)min(z + (uint32_t)u, p.splits - 1u) * p.part_stride;
#pragma unroll
                for (int i = 0; i < C; ++i) pf_load4<VEC>(pr + zo, 4u * (threadIdx.x + 256u * (uint32_t)i), p.n, q[u][i]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int i = 0; i < C; ++i)
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (z + (uint32_t)u < p.splits) a[i][c] = (z == 0 && u == 0) ? q[0][i][c] : a[i][c] + q[u][i][c];
        }
#pragma unroll
        for (int i = 0; i < C; ++i) {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[i][c] += a[i][c];
            pf_store4<VEC>(x, 4u * (threadIdx.x + 256u * (uint32_t)i), p.n, v[i]);
        }
    }
    // (elements past the row end are 0 and leave the sum unchanged)
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) ss = fmaf(v[i][c], v[i][c], ss);
    ss = block_sum<256>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)p.n + 1e-6f);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v[i][c] = (v[i][c] * inv) * gm[i][c];
            amax = fmaxf(amax, fabsf(v[i][c]));
        }
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
#pragma unroll
    for (int i = 0; i < C; ++i) pf_split4<VEC>(v[i], e, xh, xl, 4u * (threadIdx.x + 256u * (uint32_t)i), p.n);
    if (threadIdx.x == 0) p.xe[t] = e;
}

template <int EPT>
__global__ __launch_bounds__(256) void pf_rmsnorm_split_reg_kernel(PrefillRowParams p) {
    __shared__ float red[4];
    if (p.n % 4u == 0 && pf_al(p.x, 16) && pf_al(p.gamma, 8) && pf_al(p.xh, 8) && pf_al(p.xl, 8) &&
        (!p.part || (pf_al(p.part, 16) && p.part_stride % 4u == 0)))
        pf_rmsnorm_split_row<EPT, true>(p, red);
    else
        pf_rmsnorm_split_row<EPT, false>(p, red);
}

template <int EPT, bool VEC>
__device__ __forceinline__ void pf_split_row(const PrefillRowParams& p, float* red) {
    constexpr int C = EPT / 4;
    const uint32_t t = blockIdx.x;
    const float* x = p.x + (uint64_t)t * p.n;
    float v[C][4];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
        pf_load4<VEC>(x, 4u * (threadIdx.x + 256u * (uint32_t)i), p.n, v[i]);
#pragma unroll
        for (int c = 0; c < 4; ++c) amax = fmaxf(amax, fabsf(v[i][c]));
    }
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
#pragma unroll
    for (int i = 0; i < C; ++i) pf_split4<VEC>(v[i], e, xh, xl, 4u * (threadIdx.x + 256u * (uint32_t)i), p.n);
    if (threadIdx.x == 0) p.xe[t] = e;
}

template <int EPT>
__global__ __launch_bounds__(256) void pf_split_reg_kernel(PrefillRowParams p) {
    __shared__ float red[4];
    if (p.n % 4u == 0 && pf_al(p.x, 16) && pf_al(p.xh, 8) && pf_al(p.xl, 8))
        pf_split_row<EPT, true>(p, red);
    else
        pf_split_row<EPT, false>(p, red);
}

// SwiGLU rows on NT threads, thread t holding the elements t + NT i (the
// row's maximum does not depend on the thread count or order, so any NT and
// mapping give the same values; 1024 threads for 11008-wide rows: 16 waves a
// row). Loads are branch-free (indexes clamped into the row).
template <int NT, int EPT>
__global__ __launch_bounds__(NT) void pf_silu_split_reg_kernel(PrefillRowParams p) {
    __shared__ float red[NT / kWave];
    const uint32_t t = blockIdx.x;
    // p.u null: the rows already hold SiLU(g) * u (the gate|up GEMM's SwiGLU
    // pairing), only split
    const bool swiglu = p.u != nullptr;
    const float* g = p.x + (uint64_t)t * p.ld;
    const float* u = swiglu ? p.u + (uint64_t)t * p.ld : g;
    float gv[EPT], uv[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t j = min(threadIdx.x + (uint32_t)NT * (uint32_t)i, p.n - 1u);
        gv[i] = g[j];
        if (swiglu) uv[i] = u[j];
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t j = threadIdx.x + (uint32_t)NT * (uint32_t)i;
        const float h = swiglu ? (gv[i] / (1.0f + expf(-gv[i]))) * uv[i] : gv[i];
        gv[i] = j < p.n ? h : 0.f;
        amax = fmaxf(amax, fabsf(gv[i]));
    }
    const int e = pf_row_exponent(pf_block_max<NT>(amax, red));
    _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * p.n;
    _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * p.n;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t j = threadIdx.x + (uint32_t)NT * (uint32_t)i;
        if (j < p.n) pf_split(gv[i], e, xh + j, xl + j);
    }
    if (threadIdx.x == 0) p.xe[t] = e;
}

// ---------------------------------------------------------------------------
// Per-group weight exponents f_g (Q4): |s[k][g] * (q - 8)| <= 2^(eb + 3) with
// |s| <= 2^eb over the column group, so f_g = eb - 12 keeps |w'| <= 2^15.
// Two passes: blocks of 64 groups x 256 rows write the largest scale
// magnitude bits of their rows to part[row block][group]; then one thread per
// group reduces its row blocks.
// ---------------------------------------------------------------------------
constexpr uint32_t kPfExpRows = 256;

__global__ __launch_bounds__(256) void pf_weight_exp_part_kernel(const uint16_t* scales, uint32_t k, uint32_t groups,
                                                                 uint32_t* part) {
    __shared__ uint32_t red[4][kWave];
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const uint32_t g = blockIdx.x * kWave + lane;
    const uint32_t r0 = blockIdx.y * kPfExpRows, r1 = min(k, r0 + kPfExpRows);
    uint32_t mx = 0;
    if (g < groups)
        for (uint32_t r = r0 + wave; r < r1; r += 4) mx = max(mx, (uint32_t)(scales[(uint64_t)r * groups + g] & 0x7FFFu));
    red[wave][lane] = mx;
    __syncthreads();
    if (wave == 0 && g < groups)
        part[(uint64_t)blockIdx.y * groups + g] = max(max(red[0][lane], red[1][lane]), max(red[2][lane], red[3][lane]));
}

__global__ __launch_bounds__(256) void pf_weight_exp_kernel(const uint32_t* part, uint32_t nblk, uint32_t groups,
                                                            int8_t* wf) {
    const uint32_t g = blockIdx.x * 256u + threadIdx.x;
    if (g >= groups) return;
    uint32_t mx = 0;
    for (uint32_t b = 0; b < nblk; ++b) mx = max(mx, part[(uint64_t)b * groups + g]);
    const int e = (int)((mx >> 10) & 0x1F);
    const int eb = e == 0 ? -14 : e - 14;      // |s| <= 2^eb (infinities and NaN: e = 31)
    wf[g] = (int8_t)(eb - 12);
}

// ---------------------------------------------------------------------------
// The GEMM. Grid (n / NT column tiles, ceil(T / 64) token tiles).
// ---------------------------------------------------------------------------
// The K loop waits on each slice's global loads (~1 us under load) with one
// slice in flight, so what hides that latency is other blocks on the CU.
// MODE 1 (default): one LDS buffer, a second barrier per slice, 30 KB, four
// blocks per CU (512 tokens: prefill 23.4 ms). MODE 0: double-buffered LDS,
// 60 KB, two blocks per CU (26.4 ms). Two slices in flight in registers
// (141 VGPRs, two blocks per CU) measured 26.0 ms.
template <int NT, bool Q4, int MODE>
__global__ __launch_bounds__(256) void pf_gemm_kernel(PrefillGemmParams p) {
    constexpr int MT = 64, KC = 32;
    constexpr bool DB = MODE == 0;
    constexpr int NB = DB ? 2 : 1;                   // LDS buffers
    constexpr int XS = KC + 8;                      // LDS row stride in halves (80 B: 16-B aligned, no read conflicts)
    constexpr int WN = NT / 2;                      // columns per wave
    constexpr int TN = WN / 16;                     // 16-column MFMA tiles per wave
    constexpr int RPT = NT / 16;                    // weight rows per thread per slice (8 or 4)
    __shared__ __align__(16) _Float16 xs[NB][2][MT * XS];
    __shared__ __align__(16) _Float16 ws[NB][Q4 ? 2 : 1][NT * XS];

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

    // one slice of operands in registers, between its loads and its LDS stores
    struct Slice {
        uint4 xh, xl;
        uint32_t wq[RPT];                           // Q4: byte (2 columns) per row; F16: 2 halves per row
        uint16_t sc[Q4 ? RPT : 1];
    };

    auto load_slice = [&](Slice& q, uint32_t k0) {
        if (xrow_ok) {
            q.xh = *reinterpret_cast<const uint4*>(p.xh + xoff + k0);
            q.xl = *reinterpret_cast<const uint4*>(p.xl + xoff + k0);
        } else {
            q.xh = make_uint4(0, 0, 0, 0);
            q.xl = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const uint64_t row = k0 + rg * RPT + r;
            if constexpr (Q4) {
                q.wq[r] = p.w[row * (N / 2) + colc / 2];
                q.sc[r] = p.scales[row * groups + grp];
            } else {
                q.wq[r] = *reinterpret_cast<const uint32_t*>(p.w + (row * N + colc) * 2);
            }
        }
    };

    auto store_slice = [&](const Slice& q, int buf) {
        const uint4 xh_r = q.xh, xl_r = q.xl;
        const uint32_t* wq = q.wq;
        const uint16_t* sc = q.sc;
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
    const uint32_t kb = blockIdx.z * p.kper;        // this split's rows [kb, kb + steps * KC)
    const uint32_t steps = (min(K, kb + p.kper) - kb) / KC;
    auto compute = [&](int buf) {
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
    };

    Slice sa;
    load_slice(sa, kb);
    if constexpr (MODE == 0) {
        store_slice(sa, 0);
        __syncthreads();
        for (uint32_t s = 0; s < steps; ++s) {
            const int buf = (int)(s & 1u);
            if (s + 1 < steps) load_slice(sa, kb + (s + 1) * KC);
            compute(buf);
            if (s + 1 < steps) store_slice(sa, buf ^ 1);
            __syncthreads();
        }
    } else {
        for (uint32_t s = 0; s < steps; ++s) {
            if (s > 0) __syncthreads();                // every wave has read the buffer
            store_slice(sa, 0);
            __syncthreads();
            if (s + 1 < steps) load_slice(sa, kb + (s + 1) * KC);
            compute(0);
        }
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
                if (p.splits > 1) {
                    p.part[((uint64_t)blockIdx.z * p.T + row) * N + c] = v;
                } else {
                    float* y = p.y + (uint64_t)row * p.ldy + c;
                    if (p.accumulate) *y += v;
                    else *y = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill GEMM on pre-packed Q4 weights (the same numerics as pf_gemm_kernel:
// y = x' w' 2^(e_t + f_g), three f16 products per pair xh wh + xl wh + xh wl
// accumulated in fp32, in that order, per 32-deep K step).
// Block: 256 threads (4 waves) over BM tokens x 128 columns; wave w holds
// the BM x 32 output of the 32-column group w as (BM / 16) x 2 MFMA tiles.
// Only x' goes through LDS (shared by the four waves): each wave loads the
// packed weights and scales of its own columns straight into registers (a
// lane's 8 bytes are its B fragments for two tiles: 8 rows of 2 columns) and
// dequantises them there, so weights cost no LDS traffic and no second
// dequantisation (against 2 x 2 waves of BM / 2 x 64 with the weights staged
// in LDS: 72 KB of LDS traffic per block step at 64 tokens against 40 KB, and
// 20 % less time). Per K step a thread loads its x' row piece (both parts)
// and its wave's weights; loads run two steps ahead of the matrix cores,
// weights are dequantised one step ahead, and the x' LDS is double-buffered
// (one barrier per step; 16 KB a block at 64 tokens). Up to three weight
// segments share the launch (q|k|v, gate|up): column block b belongs to the
// segment whose blocks start at or below it.
//
// Packed layout (pf_pack_q4_kernel), per 128-column block nb and 32-row step
// ks: entry t = 64 rg + bc holds columns c0 = 32 (bc / 16) + bc % 16 and
// c0 + 16 (one 32-column group, so one set of scales) and rows 8 rg .. 8 rg + 7;
// lane l = 16 rg + i of the wave of group g reads entry 64 rg + 16 g + i, the
// rows and columns of its B fragments. Word c of the uint2 holds column
// c0 + 16 c: row 8 rg + 2 j in nibble j and row 8 rg + 2 j + 1 in nibble j + 4,
// so (word >> 4 j) & 0x000F000F is the pair of rows (2 j, 2 j + 1) in the low
// bits of two binary16 halves. The scales are
// stored as binary16 s' = s 2^-f_g (|s'| < 2^12), row-major per group:
// sc[((nb KS + ks) 4 + g) 32 + r]; s' is exact unless a group's scales span
// more than 2^26, where it rounds to the binary16 subnormal grid (an error
// below 2^-37 of the group's largest weight).
// Dequantisation in packed binary16: (0x6400 | q) is 1024 + q, minus 1032 is
// q - 8 (exact), times s' gives wh = f16(q' s') (one rounding of the exact
// 15-bit product, as f32 then f16 would give), and fma(q', s', -wh) gives
// wl = f16(q' s' - wh): the same wh, wl as the fp32 path, two rows at a time.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pf_pack_q4_kernel(const uint8_t* w, const uint16_t* scales, const int8_t* wf,
                                                         uint32_t k, uint32_t n, uint2* wq, uint16_t* sc) {
    // block (nb, ks): thread t packs its 16 nibbles and, for t < 128, one scale row
    const uint32_t nb = blockIdx.x, ks = blockIdx.y, KS = k / 32u;
    const uint32_t t = threadIdx.x, bc = t % 64u, rg = t / 64u;
    const uint32_t c0 = nb * 128u + (bc / 16u) * 32u + bc % 16u, c1 = c0 + 16u;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const uint32_t row = ks * 32u + rg * 8u + (uint32_t)r;
        const uint32_t b0 = w[(uint64_t)row * (n / 2u) + c0 / 2u], b1 = w[(uint64_t)row * (n / 2u) + c1 / 2u];
        const int slot = (r >> 1) + 4 * (r & 1);
        // column c is the low nibble of byte c / 2 when c is even
        w0 |= ((c0 & 1u) ? (b0 >> 4) : (b0 & 0xFu)) << (4 * slot);
        w1 |= ((c1 & 1u) ? (b1 >> 4) : (b1 & 0xFu)) << (4 * slot);
    }
    wq[((uint64_t)nb * KS + ks) * 256u + t] = make_uint2(w0, w1);
    if (t < 128u) {
        const uint32_t g = t / 32u, r = t % 32u;
        const uint16_t s = scales[(uint64_t)(ks * 32u + r) * (n / 32u) + nb * 4u + g];
        const _Float16 sv = (_Float16)(h2f(s) * ldexpf(1.0f, -(int)wf[nb * 4u + g]));
        sc[(((uint64_t)nb * KS + ks) * 4u + g) * 32u + r] = __builtin_bit_cast(uint16_t, sv);
    }
}

template <int BM>
__global__ __launch_bounds__(256, 2) void pf_gemm2_kernel(PfGemm2Params p) {
    constexpr int BN = 128, KC = 32;
    // LDS rows of 64 B (32 halves, no padding); the 16-byte chunk c of row r
    // sits at chunk c ^ ((r >> 1) & 3), which leaves the fragment reads and the
    // 64-token tiles' x' stores (four threads a row) free of bank conflicts
    constexpr int XS = KC;
    constexpr int TM = BM / 16, TN = 2;
    constexpr int XT = 256 / BM;                    // threads per x' row (8 or 4)
    constexpr int XH = KC / XT;                     // halves of a row per thread (4 or 8)
    constexpr int XV = XH / 8;                      // 16-byte loads per part (0: one 8-byte load, or 1)
    static_assert(BM == 32 || BM == 64, "32- or 64-token tiles");
    __shared__ __align__(16) _Float16 xs[2][2][BM * XS];
    kernarg_warm(p);

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const uint32_t nb = blockIdx.x;
    // the segment of this column block (wave-uniform: whole-struct selects, no
    // indexing of the argument block); with SwiGLU pairing, waves 0, 1 take
    // gate and waves 2, 3 up, each the 32-column group grp of packed block
    // lnb (h columns 64 nb + 32 (wave % 2) ..)
    const bool pair = p.swiglu != 0;
    PfGemm2Seg sg = p.seg[0];
    if (pair) {
        if (wave >= 2) sg = p.seg[1];
    } else {
        if (p.nseg > 1 && nb >= p.seg[1].nb0) sg = p.seg[1];
        if (p.nseg > 2 && nb >= p.seg[2].nb0) sg = p.seg[2];
    }
    const uint32_t lnb = pair ? nb / 2u : nb - sg.nb0;  // column block within the segment
    const uint32_t grp = pair ? 2u * (nb % 2u) + (uint32_t)wave % 2u : (uint32_t)wave;   // 32-column group in it
    const uint32_t m0 = blockIdx.y * (uint32_t)BM;
    const uint32_t K = p.k, KS = K / 32u;
    const uint32_t kb = blockIdx.z * p.kper;
    const uint32_t steps = (min(K, kb + p.kper) - kb) / (uint32_t)KC;

    // x' rows: thread t loads XH halves of row t / XT (rows past T read row T - 1, masked at the end)
    const uint32_t xr = (uint32_t)t / XT, xq = (uint32_t)t % XT;
    const uint64_t xoff = (uint64_t)min(m0 + xr, p.T - 1u) * K + xq * XH;
    // weights: lane (kq, li) of wave w holds rows 8 kq .. 8 kq + 7 of columns
    // 32 w + li and 32 w + 16 + li, with their 8 scales
    const uint32_t li = (uint32_t)lane % 16u, kq = (uint32_t)lane / 16u;
    const uint2* wqp = sg.wq + (uint64_t)lnb * KS * 256u + 64u * kq + 16u * grp + li;
    const uint16_t* scp = sg.sc + ((uint64_t)lnb * KS * 4u + grp) * 32u + 8u * kq;

    // (native vector types: the compiler keeps these in registers)
    struct Slice {
        v4u32 xh0, xl0;                             // x' pieces (32-token tiles use the first two words)
        v2u32 wq;
        v4u32 sc;                                   // 8 binary16 s', rows 8 kq .. + 7 (pairs)
    };
    auto load_slice = [&](Slice& q, uint32_t s) {
        const uint32_t k0 = kb + s * (uint32_t)KC;
        if constexpr (XV == 0) {
            const v2u32 h2 = *reinterpret_cast<const v2u32*>(p.xh + xoff + k0);
            const v2u32 l2 = *reinterpret_cast<const v2u32*>(p.xl + xoff + k0);
            q.xh0 = v4u32{h2[0], h2[1], 0u, 0u};
            q.xl0 = v4u32{l2[0], l2[1], 0u, 0u};
        } else {
            q.xh0 = *reinterpret_cast<const v4u32*>(p.xh + xoff + k0);
            q.xl0 = *reinterpret_cast<const v4u32*>(p.xl + xoff + k0);
        }
        const uint32_t ks = k0 / 32u;
        q.wq = *reinterpret_cast<const v2u32*>(wqp + (uint64_t)ks * 256u);
        q.sc = *reinterpret_cast<const v4u32*>(scp + (uint64_t)ks * 128u);
    };
    auto store_x = [&](const Slice& q, int buf) {
        if constexpr (XV == 0) {
            // half a 16-byte chunk: thread xq fills halves (xq % 2) 4 .. + 3 of chunk xq / 2
            const uint32_t xo = xr * XS + ((xq / 2u) ^ ((xr >> 1) & 3u)) * 8u + (xq % 2u) * 4u;
            *reinterpret_cast<v2u32*>(&xs[buf][0][xo]) = v2u32{q.xh0[0], q.xh0[1]};
            *reinterpret_cast<v2u32*>(&xs[buf][1][xo]) = v2u32{q.xl0[0], q.xl0[1]};
            return;
        }
        const uint32_t xc0 = xr * XS + (xq ^ ((xr >> 1) & 3u)) * 8u;
        *reinterpret_cast<v4u32*>(&xs[buf][0][xc0]) = q.xh0;
        *reinterpret_cast<v4u32*>(&xs[buf][1][xc0]) = q.xl0;
    };
    // wh, wl of the lane's two columns, two rows per binary16 pair: the B
    // fragments (k = 8 kq + b, column li) of tiles 0 and 1
    auto dequant = [&](const Slice& q, half8v* bh, half8v* bl) {
        const half2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t wv = q.wq[c];
            v4u32 wh, wl;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half2v qv = __builtin_bit_cast(half2v, ((wv >> (4 * j)) & 0x000F000Fu) | 0x64006400u) - bias;
                const uint32_t sj = q.sc[j];        // (a bit_cast of a vector element would read element 0)
                const half2v sv = __builtin_bit_cast(half2v, sj);
                const half2v h = qv * sv;
                const half2v l = __builtin_elementwise_fma(qv, sv, -h);
                wh[j] = __builtin_bit_cast(uint32_t, h);
                wl[j] = __builtin_bit_cast(uint32_t, l);
            }
            bh[c] = __builtin_bit_cast(half8v, wh);
            bl[c] = __builtin_bit_cast(half8v, wl);
        }
    };

    f32x4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // A wave raises its issue priority while it reads its fragments and issues
    // its MFMAs (64-token tiles: 3-4% faster on the large shapes, same output;
    // no effect on 32-token tiles), so the matrix cores are fed ahead of the
    // other waves' dequantisation; the compiler's MFMA/VALU interleave
    // strategy 0 adds ~1.7% there.
    auto compute = [&](int buf, const half8v* bh, const half8v* bl) {
        if constexpr (BM == 64) {
            __builtin_amdgcn_s_setprio(1);
            __builtin_amdgcn_iglp_opt(0);
        }
        half8v ah[TM], al[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const uint32_t row = (uint32_t)i * 16u + li;
            const uint32_t ch = kq ^ ((li >> 1) & 3u);     // row % 16 == li
            ah[i] = *reinterpret_cast<const half8v*>(&xs[buf][0][row * XS + ch * 8u]);
            al[i] = *reinterpret_cast<const half8v*>(&xs[buf][1][row * XS + ch * 8u]);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
            }
        if constexpr (BM == 64) __builtin_amdgcn_s_setprio(0);
    };

    // global loads run two steps ahead of the matrix cores: slice se holds the
    // even steps, so the odd ones; the LDS buffer and weight registers of step
    // s are s & 1. The steady-state loop has no branches, so the compiler
    // interleaves one step's matrix-core work with the dequantisation and LDS
    // stores of the next (loads of a clamped step index past the end stay in
    // bounds and are not used).
    Slice se, so;
    half8v bhE[TN], blE[TN], bhO[TN], blO[TN];
    if (steps > 0) {
        load_slice(se, 0);
        load_slice(so, min(1u, steps - 1u));
        store_x(se, 0);
        dequant(se, bhE, blE);
        __syncthreads();
        uint32_t s = 0;
        for (; s + 2 < steps; s += 2) {
            load_slice(se, s + 2);
            compute(0, bhE, blE);
            store_x(so, 1);
            dequant(so, bhO, blO);
            __syncthreads();
            load_slice(so, min(s + 3u, steps - 1u));
            compute(1, bhO, blO);
            store_x(se, 0);
            dequant(se, bhE, blE);
            __syncthreads();
        }
        compute(0, bhE, blE);
        if (s + 1 < steps) {
            store_x(so, 1);
            dequant(so, bhO, blO);
            __syncthreads();
            compute(1, bhO, blO);
        }
    }

    if (pair) {
        // gate waves leave their values in LDS (the x' buffers, free once
        // every wave is past its last step); up waves form h = SiLU(g) * u
        // (gemv.rs:1160-1166, the arithmetic of pf_silu_split_kernel)
        float* gt = reinterpret_cast<float*>(&xs[0][0][0]);     // [BM][64]
        static_assert(sizeof(xs) >= (size_t)BM * 64u * 4u, "gate tile fits the x' buffers");
        __syncthreads();
        if (wave < 2) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const uint32_t c = lnb * (uint32_t)BN + grp * 32u + (uint32_t)j * 16u + li;
                    const int fg = (int)sg.wf[c / 32u];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t rl = (uint32_t)i * 16u + kq * 4u + (uint32_t)r;
                        const uint32_t row = min(m0 + rl, p.T - 1u);
                        gt[rl * 64u + (uint32_t)wave * 32u + (uint32_t)j * 16u + li] = ldexpf(acc[i][j][r], p.xe[row] + fg);
                    }
                }
        }
        __syncthreads();
        if (wave < 2) return;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const uint32_t c = lnb * (uint32_t)BN + grp * 32u + (uint32_t)j * 16u + li;
                const int fg = (int)sg.wf[c / 32u];
                const uint32_t hc = 64u * nb + ((uint32_t)wave - 2u) * 32u + (uint32_t)j * 16u + li;   // h column
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t rl = (uint32_t)i * 16u + kq * 4u + (uint32_t)r;
                    const uint32_t row = m0 + rl;
                    if (row >= p.T) continue;
                    const float u = ldexpf(acc[i][j][r], p.xe[row] + fg);
                    const float g = gt[rl * 64u + ((uint32_t)wave - 2u) * 32u + (uint32_t)j * 16u + li];
                    p.seg[0].y[(uint64_t)row * p.seg[0].ldy + hc] = (g / (1.0f + expf(-g))) * u;
                }
            }
        return;
    }

    // epilogue: y = acc * 2^(e_t + f_g), stored, added, or kept as this split's partial
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t cl = (uint32_t)wave * 32u + (uint32_t)j * 16u + li;  // column in the block
            const uint32_t c = lnb * (uint32_t)BN + cl;                        // column in the segment
            const int fg = (int)sg.wf[c / 32u];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t row = m0 + (uint32_t)i * 16u + kq * 4u + (uint32_t)r;
                if (row >= p.T) continue;
                const float v = ldexpf(acc[i][j][r], p.xe[row] + fg);
                if (p.splits > 1) {
                    p.part[((uint64_t)blockIdx.z * p.T + row) * p.ntot + nb * (uint32_t)BN + cl] = v;
                } else {
                    float* y = sg.y + (uint64_t)row * sg.ldy + c;
                    if (sg.accumulate) *y += v;
                    else *y = v;
                }
            }
        }
    }
}

// Split-K partials of pf_gemm2_kernel summed in split order, stored or added
// into each segment's rows.
__global__ __launch_bounds__(256) void pf_splitk_reduce2_kernel(PfGemm2Params p) {
    const uint64_t total = (uint64_t)p.T * p.ntot;
    for (uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x; e < total; e += (uint64_t)gridDim.x * 256u) {
        float v = p.part[e];
        for (uint32_t z = 1; z < p.splits; ++z) v += p.part[(uint64_t)z * total + e];
        const uint32_t row = (uint32_t)(e / p.ntot), c = (uint32_t)(e % p.ntot);
        const uint32_t b = c / 128u;
        PfGemm2Seg sg = p.seg[0];
        if (p.nseg > 1 && b >= p.seg[1].nb0) sg = p.seg[1];
        if (p.nseg > 2 && b >= p.seg[2].nb0) sg = p.seg[2];
        float* y = sg.y + (uint64_t)row * sg.ldy + (c - sg.nb0 * 128u);
        if (sg.accumulate) *y += v;
        else *y = v;
    }
}

// Split-K partials summed in split order (deterministic), stored or added.
__global__ __launch_bounds__(256) void pf_splitk_reduce_kernel(PrefillGemmParams p) {
    const uint64_t total = (uint64_t)p.T * p.n;
    for (uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x; e < total; e += (uint64_t)gridDim.x * 256u) {
        float v = p.part[e];
        for (uint32_t z = 1; z < p.splits; ++z) v += p.part[(uint64_t)z * total + e];
        const uint64_t row = e / p.n, c = e % p.n;
        float* y = p.y + row * p.ldy + c;
        if (p.accumulate) *y += v;
        else *y = v;
    }
}

// ---------------------------------------------------------------------------
// RoPE and cache append (gemv.rs:1062-1083): q|k|v rows of tokens pos0 + t.
// q (rotated) goes to q_out [T][H][hd]; k (rotated) and v to the cache rows.
// One block per token.
// ---------------------------------------------------------------------------
template <bool F16KV>
__global__ __launch_bounds__(256) void pf_rope_cache_kernel(PrefillAttnParams p) {
    __shared__ float rs[kPfRopeRowMax];
    const uint32_t t = blockIdx.x;
    const uint32_t pos = p.pos0 + t;
    const uint32_t hd = p.hd, half = p.half;
    const uint32_t qd = p.H * hd, kvd = p.KVH * hd, qkvn = qd + 2 * kvd;
    const float* row = p.qkv + (uint64_t)t * qkvn;
    if (p.qkv_part) {
        // the q|k|v row from the GEMM's split-K partials, summed in split order
        // (as pf_splitk_reduce2_kernel would store it)
        // Four elements (i0 + 256 c) and four splits at a time, all of a
        // group's loads issued before its adds (indexes clamped into the row
        // and to the last split; the extra values are not used).
        const float* pr = p.qkv_part + (uint64_t)t * qkvn;
        for (uint32_t i0 = threadIdx.x; i0 < qkvn; i0 += 1024u) {
            float a[4];
            for (uint32_t z = 0; z < p.qkv_splits; z += 4) {
                float q[4][4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint64_t zo = (uint64_t)min(z + (uint32_t)u, p.qkv_splits - 1u) * p.qkv_part_stride;
#pragma unroll
                    for (int c = 0; c < 4; ++c) q[u][c] = pr[zo + min(i0 + 256u * (uint32_t)c, qkvn - 1u)];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (z + (uint32_t)u < p.qkv_splits) a[c] = (z == 0 && u == 0) ? q[0][c] : a[c] + q[u][c];
            }
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (i0 + 256u * (uint32_t)c < qkvn) rs[i0 + 256u * c] = a[c];
        }
        __syncthreads();
        row = rs;
    }
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
    const uint64_t cps = p.kv_ps ? p.kv_ps : kvd, chs = p.kv_ps ? p.kv_hs : hd;   // cache layout
    for (uint32_t i = threadIdx.x; i < kvd; i += 256) {
        const float kv = rotate(row + qd, i), vv = row[qd + kvd + i];
        const uint64_t idx = (uint64_t)pos * cps + (uint64_t)(i / hd) * chs + i % hd;
        if constexpr (F16KV) {
            reinterpret_cast<uint16_t*>(p.kc)[idx] = f2h(kv);
            reinterpret_cast<uint16_t*>(p.vc)[idx] = f2h(vv);
        } else {
            reinterpret_cast<float*>(p.kc)[idx] = kv;
            reinterpret_cast<float*>(p.vc)[idx] = vv;
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
// them. This VALU form covers every head shape; pf_attn_mfma_kernel below
// takes head_dim 64 or 128 with 1, 2 or 4 query heads per KV head.
// ---------------------------------------------------------------------------
template <bool F16KV>
__global__ __launch_bounds__(256) void pf_attn_vec_kernel(PrefillAttnParams p) {
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
    const uint64_t cps = p.kv_ps ? p.kv_ps : kvd, chs = p.kv_ps ? p.kv_hs : hd;   // cache layout
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
            const uint64_t idx = (uint64_t)kp * cps + (uint64_t)kvh * chs + d;
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

// ---------------------------------------------------------------------------
// Causal prefill attention on the matrix cores. Block (query tile, KV head),
// 4 waves; wave w takes query head kvh * G + w % G for 16 queries (sub-tile
// w / G), so the G heads sharing a KV head share each K/V tile staged in LDS
// (64 keys per step). Per wave and key tile:
//   * S^T = K Q^T on the f16 matrix cores (v_mfma_f32_16x16x32_f16), K from
//     LDS as the A operand and Q held in registers as B, each split into two
//     binary16 parts on a power-of-two scale (per key row, per query: as the
//     prefill GEMM splits its operands; 22-bit products, fp32 accumulation),
//     the dot then scaled back exactly. Lane (g, i) holds the scores of
//     query i for keys 16 c + 4 g + r (c, r < 4): the online softmax of a
//     query runs in its own four lanes and its probabilities never leave them;
//   * O^T += V^T P^T on the f16 matrix cores (v_mfma_f32_16x16x32_f16), both
//     operands split into two binary16 parts, three products (vh ph + vl ph +
//     vh pl) accumulated in fp32. The contraction runs over the 32 keys of a
//     half tile in the order lane group g holds them: position 8 g + b is key
//     16 (b / 4) + 4 g + b % 4, so P^T comes straight from the lane's
//     probabilities and V is staged as VT[s][g][d][8] binary16 (the 8 keys a
//     lane needs for dim d, contiguous).
// Precision: products of the f16 parts are exact; p and v are held to 22
// bits above 2^-14 (below, to an absolute 2^-25: p <= 1, and a value that
// small moves the sum by less than fp32 rounding of the larger terms).
// Operand layouts of v_mfma_f32_16x16x32_f16 (lane l): A[i = l % 16][k =
// 8 (l / 16) + b], B[k = 8 (l / 16) + b][j = l % 16], C[i = 4 (l / 16) + r]
// [j = l % 16] in register r.
// ---------------------------------------------------------------------------
template <int HD, bool F16KV>
__global__ __launch_bounds__(256, 2) void pf_attn_mfma_kernel(PrefillAttnParams p) {
    constexpr int KT = 64;                          // keys per step
    constexpr int QC = HD / 32;                     // 32-deep contraction steps of K Q^T
    constexpr int OC = HD / 16;                     // 16-dim output tiles
    // K of the tile: kt[part][step st][key][32 dims] binary16 (dims 32 st ..),
    // 16-byte chunk c of key r at chunk c ^ ((r >> 1) & 3); ksc[key] = 2^e_k
    __shared__ __align__(16) _Float16 kt[2][QC][KT * 32];
    __shared__ __align__(16) float ksc[KT];
    // V of the tile: vt[part][half s][lane group g][dim d][8 keys], binary16
    __shared__ __align__(16) _Float16 vt[2][2 * 4 * HD * 8];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t % kWave, g4 = lane / 16u, li = lane % 16u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const uint32_t G = p.H / p.KVH, kvh = blockIdx.y;
    const uint32_t sub = wave / G;                  // query sub-tile of this wave
    const uint32_t h = kvh * G + wave % G;
    const uint32_t QT = 16u * (4u / G);             // queries per block
    const uint32_t nc = p.nc > 1u ? p.nc : 1u;      // key chunks per query block
    const uint32_t q0 = (blockIdx.x / nc) * QT;     // chunk-relative first query of the block
    const uint32_t qd = p.H * HD, kvd = p.KVH * HD;
    const uint64_t cps = p.kv_ps ? p.kv_ps : kvd, chs = p.kv_ps ? p.kv_hs : HD;   // cache layout
    const uint32_t nq = min(QT, p.T - q0);
    const uint32_t last = p.pos0 + q0 + nq - 1u;    // last key any query of the block needs
    const uint32_t wq0 = q0 + sub * 16u;            // this wave's first query
    const bool wave_on = sub * 16u < nq;            // waves of a partial tile may hold no query
    // this block's keys [kbeg, kend): all of them, or key chunk blockIdx.x % nc
    const uint32_t kbeg = nc > 1u ? (blockIdx.x % nc) * p.ch : 0u;
    const uint32_t kend = nc > 1u ? min(kbeg + p.ch, last + 1u) : last + 1u;
    if (kbeg > last) return;                        // a chunk past every key of the block

    // Q fragment (B operand of K Q^T): lane holds q[wq0 + li][32 st + 8 g4 + b]
    // times 2^-e_q (e_q from the query's max |q|: the lane's four-lane group)
    // as two binary16 parts
    half8v qh[QC], ql[QC];
    float sq;                                       // 2^e_q
    {
        const uint32_t qi = min(wq0 + li, p.T - 1u);
        const float* qrow = p.q + (uint64_t)qi * qd + (uint64_t)h * HD + 8u * g4;
        float qv[QC][8];
        float amax = 0.f;
#pragma unroll
        for (int st = 0; st < QC; ++st) {
            const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * st);
            const float4 b = *reinterpret_cast<const float4*>(qrow + 32 * st + 4);
            qv[st][0] = a.x; qv[st][1] = a.y; qv[st][2] = a.z; qv[st][3] = a.w;
            qv[st][4] = b.x; qv[st][5] = b.y; qv[st][6] = b.z; qv[st][7] = b.w;
#pragma unroll
            for (int b8 = 0; b8 < 8; ++b8) amax = fmaxf(amax, fabsf(qv[st][b8]));
        }
        amax = max_row_slots(amax);
        const int eq = pf_row_exponent(amax);
        sq = ldexpf(1.0f, eq);
#pragma unroll
        for (int st = 0; st < QC; ++st)
#pragma unroll
            for (int b8 = 0; b8 < 8; ++b8) {
                const float v = ldexpf(qv[st][b8], -eq);
                const _Float16 hv = (_Float16)v;
                qh[st][b8] = hv;
                ql[st][b8] = (_Float16)(v - (float)hv);
            }
    }
    const uint32_t qpos = p.pos0 + wq0 + li;        // this lane's query position
    // scores in log2 units: dot * 2^(e_k + e_q) * scale * log2(e), so the
    // softmax runs on v_exp_f32 (2^x) directly; m leaves as m ln 2
    const float qf = sq * p.scale * 1.4426950408889634f;
    float m = -INFINITY, l = 0.f;
    f32x4v o[OC];
#pragma unroll
    for (int c = 0; c < OC; ++c) o[c] = f32x4v{0.f, 0.f, 0.f, 0.f};

    // A tile's K and V are loaded into registers one tile ahead (thread e of
    // the K load: key e / (HD/4), dims 4 (e % (HD/4)) ..; of the V load: dim
    // e % HD, keys 4 (e / HD) .. + 3), then staged in LDS.
    constexpr int KE = KT * HD / 4 / 256;           // K float4s per thread
    constexpr int VE = HD * KT / 4 / 256;           // V key quads per thread
    float4 kreg[KE];
    float vreg[VE][4];
    // Cache rows addressed from the KV head's base (uniform) by 32-bit byte
    // offsets row * row_bytes + column bytes (24-bit multiplies) when every
    // offset of the block fits; 64-bit element indexes otherwise.
    constexpr uint32_t ES = F16KV ? 2u : 4u;
    const bool off32 = last < (1u << 24) && cps * ES < (1u << 24) &&
                       ((uint64_t)last + 1u) * cps * ES + (uint64_t)HD * ES < (1ull << 31);
    const char* kbase = reinterpret_cast<const char*>(p.kc) + (uint64_t)kvh * chs * ES;
    const char* vbase = reinterpret_cast<const char*>(p.vc) + (uint64_t)kvh * chs * ES;
    const uint32_t rowb = (uint32_t)(cps * ES);
    auto load_tile = [&](uint32_t k0) {
        if (off32) {
#pragma unroll
            for (int u = 0; u < KE; ++u) {
                const uint32_t e = t + 256u * (uint32_t)u;
                const uint32_t r = e / (HD / 4), c4 = e % (HD / 4);
                const uint32_t o = __umul24(min(k0 + r, last), rowb) + 4u * c4 * ES;
                if constexpr (F16KV) {
                    const uint2 a = *reinterpret_cast<const uint2*>(kbase + o);
                    kreg[u] = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), 0.f, 0.f);   // raw words
                } else {
                    kreg[u] = *reinterpret_cast<const float4*>(kbase + o);
                }
            }
#pragma unroll
            for (int u = 0; u < VE; ++u) {
                const uint32_t e = t + 256u * (uint32_t)u;
                const uint32_t d = e % HD, quad = e / HD;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const uint32_t o = __umul24(min(k0 + 4u * quad + (uint32_t)rr, last), rowb) + d * ES;
                    if constexpr (F16KV) vreg[u][rr] = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(vbase + o));
                    else vreg[u][rr] = *reinterpret_cast<const float*>(vbase + o);
                }
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < KE; ++u) {
            const uint32_t e = t + 256u * (uint32_t)u;
            const uint32_t r = e / (HD / 4), c4 = e % (HD / 4);
            const uint64_t idx = (uint64_t)min(k0 + r, last) * cps + (uint64_t)kvh * chs + 4u * c4;
            if constexpr (F16KV) {
                const uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p.kc) + idx);
                kreg[u] = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), 0.f, 0.f);   // raw words
            } else {
                kreg[u] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.kc) + idx);
            }
        }
#pragma unroll
        for (int u = 0; u < VE; ++u) {
            const uint32_t e = t + 256u * (uint32_t)u;
            const uint32_t d = e % HD, quad = e / HD;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const uint64_t idx = (uint64_t)min(k0 + 4u * quad + (uint32_t)rr, last) * cps + (uint64_t)kvh * chs + d;
                if constexpr (F16KV) vreg[u][rr] = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p.vc)[idx]);
                else vreg[u][rr] = reinterpret_cast<const float*>(p.vc)[idx];
            }
        }
    };
    typedef _Float16 half4v __attribute__((ext_vector_type(4)));
    auto store_tile = [&]() {
        // K: key r's HD/4 threads (consecutive lanes) share its exponent e_k
        // (max |k| of the row, butterfly over those lanes), then two binary16 parts
#pragma unroll
        for (int u = 0; u < KE; ++u) {
            const uint32_t e = t + 256u * (uint32_t)u;
            const uint32_t r = e / (HD / 4), c4 = e % (HD / 4);
            float4 kv = kreg[u];
            if constexpr (F16KV) {
                const uint32_t ax = __float_as_uint(kv.x), ay = __float_as_uint(kv.y);
                kv = make_float4(h2f((uint16_t)(ax & 0xFFFFu)), h2f((uint16_t)(ax >> 16)),
                                 h2f((uint16_t)(ay & 0xFFFFu)), h2f((uint16_t)(ay >> 16)));
            }
            const float amax = group_max<HD / 4>(fmaxf(fmaxf(fabsf(kv.x), fabsf(kv.y)), fmaxf(fabsf(kv.z), fabsf(kv.w))));
            const int ek = pf_row_exponent(amax);
            const float kin[4] = {ldexpf(kv.x, -ek), ldexpf(kv.y, -ek), ldexpf(kv.z, -ek), ldexpf(kv.w, -ek)};
            _Float16 kh[4], kl[4];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                kh[q4] = (_Float16)kin[q4];
                kl[q4] = (_Float16)(kin[q4] - (float)kh[q4]);
            }
            const uint32_t st = c4 / 8u, ch = ((c4 % 8u) / 2u) ^ ((r >> 1) & 3u);
            const uint32_t o4 = r * 32u + ch * 8u + (c4 % 2u) * 4u;
            *reinterpret_cast<half4v*>(&kt[0][st][o4]) = half4v{kh[0], kh[1], kh[2], kh[3]};
            *reinterpret_cast<half4v*>(&kt[1][st][o4]) = half4v{kl[0], kl[1], kl[2], kl[3]};
            if (c4 == 0) ksc[r] = ldexpf(1.0f, ek);
        }
#pragma unroll
        for (int u = 0; u < VE; ++u) {
            const uint32_t e = t + 256u * (uint32_t)u;
            const uint32_t d = e % HD, quad = e / HD;   // keys 4 quad .. 4 quad + 3
            const uint32_t hs = quad / 8u, cq = (quad % 8u) / 4u, gq = quad % 4u;
            _Float16 vh[4], vl[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const float v = F16KV ? h2f((uint16_t)__float_as_uint(vreg[u][rr])) : vreg[u][rr];
                vh[rr] = (_Float16)v;
                vl[rr] = (_Float16)(v - (float)vh[rr]);
            }
            const uint32_t o8 = ((hs * 4u + gq) * (uint32_t)HD + d) * 8u + cq * 4u;
            *reinterpret_cast<half4v*>(&vt[0][o8]) = half4v{vh[0], vh[1], vh[2], vh[3]};
            *reinterpret_cast<half4v*>(&vt[1][o8]) = half4v{vl[0], vl[1], vl[2], vl[3]};
        }
    };

    load_tile(kbeg);
    for (uint32_t k0 = kbeg; k0 < kend; k0 += KT) {
        __syncthreads();                            // the previous tiles are consumed
        store_tile();
        __syncthreads();
        // the next tile's loads (clamped: past the last key they re-read it)
        load_tile(k0 + KT < kend ? k0 + KT : k0);
        // a wave with no visible key in the tile skips the work, not the barriers
        if (!(wave_on && k0 <= p.pos0 + wq0 + 15u)) continue;
        // ---- S^T = K Q^T: four 16-key x 16-query tiles, three binary16 products
        // (kh qh + kl qh + kh ql) per 32-deep step ----
        f32x4v sacc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            sacc[c] = f32x4v{0.f, 0.f, 0.f, 0.f};
            const uint32_t o8 = (16u * c + li) * 32u + (g4 ^ ((li >> 1) & 3u)) * 8u;
#pragma unroll
            for (int st = 0; st < QC; ++st) {
                const half8v kh = *reinterpret_cast<const half8v*>(&kt[0][st][o8]);
                const half8v kl = *reinterpret_cast<const half8v*>(&kt[1][st][o8]);
                sacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[st], sacc[c], 0, 0, 0);
                sacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[st], sacc[c], 0, 0, 0);
                sacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[st], sacc[c], 0, 0, 0);
            }
        }
        // ---- online softmax of query li over keys 16 c + 4 g4 + r ----
        float sv[4][4];
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 kf = *reinterpret_cast<const float4*>(&ksc[16u * c + 4u * g4]);
            const float kfa[4] = {kf.x, kf.y, kf.z, kf.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t kp = k0 + 16u * c + 4u * g4 + (uint32_t)r;
                sv[c][r] = kp <= qpos ? sacc[c][r] * (kfa[r] * qf) : -INFINITY;
                mx = fmaxf(mx, sv[c][r]);
            }
        }
        mx = max_row_slots(mx);
        const float m_new = fmaxf(m, mx);
        const float mref = m_new == -INFINITY ? 0.f : m_new;   // a query with no visible key yet
        const float f = __builtin_amdgcn_exp2f(m - mref);
        float sum = 0.f;
        half8v ph[2], pl[2];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(sv[c][r] - mref);
                sum += e;
                const _Float16 eh = (_Float16)e;
                ph[c / 2][(c % 2) * 4 + r] = eh;
                pl[c / 2][(c % 2) * 4 + r] = (_Float16)(e - (float)eh);
            }
        sum = sum_row_slots(sum);
        l = l * f + sum;
        m = m_new;
        // ---- O^T = O^T f + V^T P^T: dim tiles of 16, two half tiles of 32 keys ----
#pragma unroll
        for (int c = 0; c < OC; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[c][r] *= f;
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
#pragma unroll
            for (int c = 0; c < OC; ++c) {
                const uint32_t o8 = (((uint32_t)hs * 4u + g4) * (uint32_t)HD + 16u * c + li) * 8u;
                const half8v ah = *reinterpret_cast<const half8v*>(&vt[0][o8]);
                const half8v al = *reinterpret_cast<const half8v*>(&vt[1][o8]);
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, ph[hs], o[c], 0, 0, 0);
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, ph[hs], o[c], 0, 0, 0);
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, pl[hs], o[c], 0, 0, 0);
            }
        }
    }
    if (!wave_on) return;
    // lane (g4, li): O^T[dims 16 c + 4 g4 + r][query li]
    const uint32_t row = li;                        // query within the wave's 16
    if (wq0 + row >= q0 + nq) return;
    if (nc > 1u) {
        // partial state of the chunk: unnormalised o, running max m and sum l
        // per row, merged by pf_attn_merge_kernel / pf_attn_merge_split_kernel
        const uint64_t blk = (uint64_t)blockIdx.x * p.KVH + kvh;
        float* po = p.part + (blk * 64u + wave * 16u) * HD;
        float* pml = p.part + (uint64_t)gridDim.x * p.KVH * 64u * HD + (blk * 64u + wave * 16u) * 2u;
#pragma unroll
        for (int c = 0; c < OC; ++c)
            *reinterpret_cast<float4*>(&po[row * HD + 16 * c + 4 * g4]) = make_float4(o[c][0], o[c][1], o[c][2], o[c][3]);
        if (g4 == 0) {
            pml[row * 2u] = m * 0.6931471805599453f;   // natural units for the merge
            pml[row * 2u + 1u] = l;
        }
        return;
    }
    const float inv = 1.0f / l;
    float* out = p.out + (uint64_t)(wq0 + row) * qd + (uint64_t)h * HD;
#pragma unroll
    for (int c = 0; c < OC; ++c)
        *reinterpret_cast<float4*>(&out[16 * c + 4 * g4]) =
            make_float4(o[c][0] * inv, o[c][1] * inv, o[c][2] * inv, o[c][3] * inv);
}

// Merge of the key chunks of pf_attn_mfma_kernel (nc > 1): blocks of 256
// elements of a token row; out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c over the chunks
// holding keys of the row's query block (a chunk with no key visible to the
// row has m = -inf and adds nothing).
template <int HD>
__global__ __launch_bounds__(256) void pf_attn_merge_kernel(PrefillAttnParams p) {
    constexpr uint32_t MC = 8;                      // most chunks (the workspace's bound)
    const uint32_t t = blockIdx.x;
    const uint32_t G = p.H / p.KVH, QT = 16u * (4u / G), nc = p.nc;
    const uint32_t qb = t / QT, qloc = t % QT, sub = qloc / 16u, row = qloc % 16u;
    const uint32_t q0 = qb * QT, nq = min(QT, p.T - q0);
    const uint32_t last = p.pos0 + q0 + nq - 1u;
    const uint32_t nlive = min(min(nc, MC), last / p.ch + 1u);
    const uint64_t nblk = (uint64_t)((p.T + QT - 1u) / QT) * nc * p.KVH;
    const float* po = p.part;
    const float* pml = p.part + nblk * 64u * HD;
    const uint32_t qd = p.H * HD;
    // thread: element e = head * HD + d of the row (grid.y covers the row in
    // 256-element pieces); every chunk's (m, l, o) requested before any is used
    const uint32_t e = blockIdx.y * 256u + threadIdx.x;
    if (e < qd) {
        const uint32_t h = e / HD, d = e % HD;
        const uint32_t kvh = h / G, wave = sub * G + h % G;
        float mv[MC], lv[MC], ov[MC];
#pragma unroll
        for (uint32_t kc = 0; kc < MC; ++kc) {
            const uint32_t kk = min(kc, nlive - 1u);
            const uint64_t r = (((uint64_t)qb * nc + kk) * p.KVH + kvh) * 64u + wave * 16u + row;
            mv[kc] = pml[r * 2u];
            lv[kc] = pml[r * 2u + 1u];
            ov[kc] = po[r * HD + d];
        }
        float M = mv[0];
#pragma unroll
        for (uint32_t kc = 1; kc < MC; ++kc) M = fmaxf(M, mv[kc]);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (uint32_t kc = 0; kc < MC; ++kc) {
            if (kc >= nlive) break;
            const float w = expf(mv[kc] - M);
            num = fmaf(w, ov[kc], num);
            den = fmaf(w, lv[kc], den);
        }
        p.out[(uint64_t)t * qd + h * HD + d] = num / den;
    }
}

// pf_attn_merge_kernel and pf_split_kernel in one pass: block t merges row
// t's key chunks (thread: 8 consecutive dims of one head; the same per-element
// arithmetic, in the same chunk order) and splits the row for the o GEMM.
template <int HD>
__global__ __launch_bounds__(256) void pf_attn_merge_split_kernel(PrefillAttnParams p) {
    constexpr uint32_t MC = 8;                      // most chunks (the workspace's bound)
    constexpr uint32_t DPT = 8;                     // dims per thread
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    const uint32_t G = p.H / p.KVH, QT = 16u * (4u / G), nc = p.nc;
    const uint32_t qb = t / QT, qloc = t % QT, sub = qloc / 16u, row = qloc % 16u;
    const uint32_t q0 = qb * QT, nq = min(QT, p.T - q0);
    const uint32_t last = p.pos0 + q0 + nq - 1u;
    const uint32_t nlive = min(min(nc, MC), last / p.ch + 1u);
    const uint64_t nblk = (uint64_t)((p.T + QT - 1u) / QT) * nc * p.KVH;
    const float* po = p.part;
    const float* pml = p.part + nblk * 64u * HD;
    const uint32_t qd = p.H * HD;
    const uint32_t e0 = threadIdx.x * DPT;          // first element of the row (qd <= 256 DPT)
    const bool on = e0 < qd;
    const uint32_t h = min(e0, qd - 1u) / HD, d0 = min(e0, qd - 1u) % HD;
    const uint32_t kvh = h / G, wave = sub * G + h % G;
    float mv[MC], lv[MC], ov[MC][DPT];
#pragma unroll
    for (uint32_t kc = 0; kc < MC; ++kc) {
        const uint32_t kk = min(kc, nlive - 1u);
        const uint64_t r = (((uint64_t)qb * nc + kk) * p.KVH + kvh) * 64u + wave * 16u + row;
        mv[kc] = pml[r * 2u];
        lv[kc] = pml[r * 2u + 1u];
        const float4 a = *reinterpret_cast<const float4*>(po + r * HD + d0);
        const float4 b = *reinterpret_cast<const float4*>(po + r * HD + d0 + 4u);
        ov[kc][0] = a.x; ov[kc][1] = a.y; ov[kc][2] = a.z; ov[kc][3] = a.w;
        ov[kc][4] = b.x; ov[kc][5] = b.y; ov[kc][6] = b.z; ov[kc][7] = b.w;
    }
    float M = mv[0];
#pragma unroll
    for (uint32_t kc = 1; kc < MC; ++kc) M = fmaxf(M, mv[kc]);
    float num[DPT], den = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < DPT; ++i) num[i] = 0.f;
#pragma unroll
    for (uint32_t kc = 0; kc < MC; ++kc) {
        if (kc >= nlive) break;
        const float w = expf(mv[kc] - M);
#pragma unroll
        for (uint32_t i = 0; i < DPT; ++i) num[i] = fmaf(w, ov[kc][i], num[i]);
        den = fmaf(w, lv[kc], den);
    }
    float v[DPT], amax = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < DPT; ++i) {
        v[i] = num[i] / den;
        amax = on ? fmaxf(amax, fabsf(v[i])) : amax;
    }
    const int e = pf_row_exponent(pf_block_max<256>(amax, red));
    if (on) {
        _Float16* xh = reinterpret_cast<_Float16*>(p.xh) + (uint64_t)t * qd + e0;
        _Float16* xl = reinterpret_cast<_Float16*>(p.xl) + (uint64_t)t * qd + e0;
        if (pf_al(xh, 16) && pf_al(xl, 16)) {
            half8v hv, lv8;
#pragma unroll
            for (uint32_t i = 0; i < DPT; ++i) {
                const float sv = ldexpf(v[i], -e);
                hv[i] = (_Float16)sv;
                lv8[i] = (_Float16)(sv - (float)hv[i]);
            }
            *reinterpret_cast<half8v*>(xh) = hv;
            *reinterpret_cast<half8v*>(xl) = lv8;
        } else {
#pragma unroll
            for (uint32_t i = 0; i < DPT; ++i) pf_split(v[i], e, xh + i, xl + i);
        }
    }
    if (threadIdx.x == 0) p.xe[t] = e;
}

}  // namespace qora
