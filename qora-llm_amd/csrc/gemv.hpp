// Batch-1 GEMV kernels for the QORA weight formats on gfx950.
//
// Projection layout (the reference's Q4Weight / F16Weight, gemv.rs:23-38):
//   Q4 : packed[k][n/2] bytes, low nibble = even column, q in [0,15],
//        value = (q - 8) * scale; scales[k][n/32] binary16.
//   F16: data[k][n] binary16.
// y[j] = sum_i x[i] * W[i][j]  (outer-product form of gemv_q4, gemv.rs:596-675).
//
// Work decomposition (split-K, no atomics on the result):
//   * A "group" is 32 output columns of one input row: 16 bytes of nibbles
//     plus one scale (Q4), or 64 bytes (F16). Each lane owns one group and
//     accumulates its 32 columns in registers over RPL rows, so one 128-bit
//     load feeds 32 multiply-adds.
//   * A workgroup (256 lanes) covers a column tile of GT groups and a slice of
//     KR = (256/GT)*RPL input rows. Lanes t = rl*GT + gi: the GT lanes of a
//     row read GT*16 contiguous bytes, so every wave instruction reads 64/GT
//     full row segments (128 B or 256 B each).
//   * Lanes sharing a group are summed through LDS; the workgroup writes one
//     partial per column. The last workgroup to finish a column tile (device
//     scope counter) adds the S partials in split order, which makes the
//     result independent of scheduling, and runs the epilogue.
// Segments: up to three weight matrices are addressed as one virtual matrix
// (q|k|v concatenated by column tiles), or two matrices are paired lane by
// lane (gate|up) so the SiLU*up epilogue finds both halves in one workgroup.
// The weights are read in the reference layout; nothing is repacked.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace qora {




__device__ __forceinline__ float silu_mul(float g, float u) {
    const float silu_g = g / (1.0f + expf(-g));
    return silu_g * u;
}

template <int FMT, int GT, int RPL>
__global__ __launch_bounds__(256) void gemv_splitk_kernel(GemvParams p) {
    constexpr int NT = 256;
    constexpr int RL = NT / GT;          // row lanes
    constexpr int COLS = GT * 32;        // columns per tile
    constexpr int KR = RL * RPL;         // rows per workgroup
    constexpr int RED_STRIDE = 33;       // padded group stride in LDS
    constexpr int CPT = COLS / NT;       // columns per thread in the reduction

    __shared__ float xs[KR];
    __shared__ float red[NT * RED_STRIDE];
    __shared__ float wred[NT / kWave];
    __shared__ int s_last;

    const int t = threadIdx.x;
    const int gi = t % GT;
    const int rl = t / GT;
    const uint32_t tile = blockIdx.x % p.tiles;
    const uint32_t split = blockIdx.x / p.tiles;
    const uint32_t k0 = split * p.rows_per_split;
    const uint32_t k1 = min(p.k, k0 + p.rows_per_split);

    // ---- prologue: stage x[k0, k1) (optionally RMS-normalised) in LDS ----
    float inv_rms = 1.0f;
    if (p.gamma) {
        float ss = 0.f;
        for (uint32_t i = t; i < p.k; i += NT) { const float v = p.x[i]; ss += v * v; }
        ss = block_sum<NT>(ss, wred);
        inv_rms = 1.0f / sqrtf(ss / (float)p.k + 1e-6f);
    }
    for (int i = t; i < KR; i += NT) {
        const uint32_t r = k0 + i;
        float v = 0.f;
        if (r < k1) {
            v = p.x[r];
            if (p.gamma) v = v * inv_rms * h2f(p.gamma[r]);
        }
        xs[i] = v;
    }

    // ---- which segment / group this lane reads ----
    int sidx;
    uint32_t grp;
    if (p.paired) {
        sidx = gi < GT / 2 ? 0 : 1;
        grp = tile * (GT / 2) + (gi % (GT / 2));
    } else {
        sidx = 0;
        if (p.nseg > 1 && tile >= p.seg[1].tile0) sidx = 1;
        if (p.nseg > 2 && tile >= p.seg[2].tile0) sidx = 2;
        grp = (tile - p.seg[sidx].tile0) * GT + gi;
    }
    const GemvSeg sg = p.seg[sidx];
    const bool active = grp < sg.groups;

    __syncthreads();

    float acc[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[c] = 0.f;

    if constexpr (FMT == FMT_Q4) {
        const uint64_t row_bytes = (uint64_t)sg.groups * 16u;
        uint4 wv[RPL];
        uint16_t sv[RPL];
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const uint32_t r = k0 + rl + j * RL;
            if (active && r < k1) {
                wv[j] = *reinterpret_cast<const uint4*>(sg.w + r * row_bytes + (uint64_t)grp * 16u);
                sv[j] = sg.scales[(uint64_t)r * sg.groups + grp];
            } else {
                wv[j] = make_uint4(0, 0, 0, 0);
                sv[j] = 0;
            }
        }
        float corr = 0.f;
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const float sx = h2f(sv[j]) * xs[rl + j * RL];
            corr += sx;
            const uint32_t w4[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t lo = w4[d] & 0x0F0F0F0Fu;
                const uint32_t hi = (w4[d] >> 4) & 0x0F0F0F0Fu;
                acc[d * 8 + 0] = fmaf(sx, ubyte_f<0>(lo), acc[d * 8 + 0]);
                acc[d * 8 + 1] = fmaf(sx, ubyte_f<0>(hi), acc[d * 8 + 1]);
                acc[d * 8 + 2] = fmaf(sx, ubyte_f<1>(lo), acc[d * 8 + 2]);
                acc[d * 8 + 3] = fmaf(sx, ubyte_f<1>(hi), acc[d * 8 + 3]);
                acc[d * 8 + 4] = fmaf(sx, ubyte_f<2>(lo), acc[d * 8 + 4]);
                acc[d * 8 + 5] = fmaf(sx, ubyte_f<2>(hi), acc[d * 8 + 5]);
                acc[d * 8 + 6] = fmaf(sx, ubyte_f<3>(lo), acc[d * 8 + 6]);
                acc[d * 8 + 7] = fmaf(sx, ubyte_f<3>(hi), acc[d * 8 + 7]);
            }
        }
        // sum_r sx_r*(q-8) = sum_r sx_r*q - 8*sum_r sx_r
#pragma unroll
        for (int c = 0; c < 32; ++c) acc[c] = fmaf(-8.0f, corr, acc[c]);
    } else {
        const uint64_t row_bytes = (uint64_t)sg.groups * 64u;
        constexpr int B = RPL < 4 ? RPL : 4;   // rows of 64 B in flight per batch
#pragma unroll
        for (int j0 = 0; j0 < RPL; j0 += B) {
            uint4 wv[B][4];
#pragma unroll
            for (int j = 0; j < B; ++j) {
                const uint32_t r = k0 + rl + (j0 + j) * RL;
                if (active && r < k1) {
                    const uint4* src = reinterpret_cast<const uint4*>(sg.w + r * row_bytes + (uint64_t)grp * 64u);
#pragma unroll
                    for (int v = 0; v < 4; ++v) wv[j][v] = src[v];
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v) wv[j][v] = make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < B; ++j) {
                const float xr = xs[rl + (j0 + j) * RL];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t w4[4] = {wv[j][v].x, wv[j][v].y, wv[j][v].z, wv[j][v].w};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        acc[v * 8 + d * 2 + 0] = fmaf(xr, h2f((uint16_t)(w4[d] & 0xFFFFu)), acc[v * 8 + d * 2 + 0]);
                        acc[v * 8 + d * 2 + 1] = fmaf(xr, h2f((uint16_t)(w4[d] >> 16)), acc[v * 8 + d * 2 + 1]);
                    }
                }
            }
        }
    }

    // ---- reduce the RL row lanes of each group through LDS ----
    {
        float* dst = red + (rl * GT + gi) * RED_STRIDE;
#pragma unroll
        for (int c = 0; c < 32; ++c) dst[c] = acc[c];
    }
    __syncthreads();
    float colv[CPT];
#pragma unroll
    for (int cc = 0; cc < CPT; ++cc) {
        const int col = t + cc * NT;
        const int g = col / 32, c = col % 32;
        float s = 0.f;
#pragma unroll 8
        for (int r = 0; r < RL; ++r) s += red[(r * GT + g) * RED_STRIDE + c];
        colv[cc] = s;
    }

    if (p.splits > 1) {
        float* dst = p.partials + ((uint64_t)split * p.tiles + tile) * COLS;
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) dst[t + cc * NT] = colv[cc];
        __threadfence();
        __syncthreads();
        if (t == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_ACQ_REL,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            s_last = (prev == p.splits - 1) ? 1 : 0;
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) {
            const int col = t + cc * NT;
            float s = 0.f;
            for (uint32_t q = 0; q < p.splits; ++q)
                s += p.partials[((uint64_t)q * p.tiles + tile) * COLS + col];
            colv[cc] = s;
        }
        if (t == 0) store_u32_release(&p.counters[tile], 0u);
    }

    // ---- epilogue on the final column sums ----
    if (p.epi == EPI_STORE || p.epi == EPI_RESID) {
        // single segment, plain layout
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) {
            const uint32_t col = tile * COLS + t + cc * NT;
            if (col < p.seg[0].groups * 32u) {
                if (p.epi == EPI_STORE) p.y[col] = colv[cc];
                else p.y[col] += colv[cc];
            }
        }
        return;
    }
    __syncthreads();  // red[] reused as the staging buffer below
    float* sums = red;
#pragma unroll
    for (int cc = 0; cc < CPT; ++cc) sums[t + cc * NT] = colv[cc];
    __syncthreads();
    if (p.epi == EPI_SILU) {
        constexpr int HALF = COLS / 2;
        const uint32_t n = p.seg[0].groups * 32u;
        for (int c = t; c < HALF; c += NT) {
            const uint32_t j = tile * HALF + c;
            if (j < n) p.y[j] = silu_mul(sums[c], sums[c + HALF]);
        }
        return;
    }
    // EPI_QKV: segment 0 -> q, 1 -> K cache row, 2 -> V cache row.
    {
        const int s = (p.nseg > 2 && tile >= p.seg[2].tile0) ? 2 : ((tile >= p.seg[1].tile0) ? 1 : 0);
        const uint32_t seg_cols = p.seg[s].groups * 32u;
        const uint32_t base = (tile - p.seg[s].tile0) * COLS;
        const int32_t pos = *p.pos;
        const uint32_t hd = p.head_dim, half = p.half_dim;
        for (int c = t; c < COLS; c += NT) {
            const uint32_t lc = base + c;
            if (lc >= seg_cols) continue;
            float v = sums[c];
            if (s < 2 && p.use_rope) {
                // apply_rope_raw (gemv.rs:757-778): pairs (i, i+half) in each head
                const uint32_t d = lc % hd;
                const float* ct = p.rope_cos + (uint64_t)pos * half;
                const float* st = p.rope_sin + (uint64_t)pos * half;
                if (d < half) {
                    const float x1 = v, x2 = sums[c + half];
                    v = x1 * ct[d] - x2 * st[d];
                } else if (d < 2 * half) {
                    const float x1 = sums[c - half], x2 = v;
                    v = x2 * ct[d - half] + x1 * st[d - half];
                }
            }
            if (s == 0) {
                p.q_out[lc] = v;
            } else {
                void* cache = (s == 1) ? p.kcache : p.vcache;
                const uint64_t idx = (uint64_t)pos * p.kv_stride + lc;
                if (p.kv_f16) reinterpret_cast<uint16_t*>(cache)[idx] = f2h(v);
                else reinterpret_cast<float*>(cache)[idx] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row-dot GEMV over a [rows][cols] matrix (the tied lm_head,
// lm_head_parallel_q4 / _f16, gemv.rs:805-864): y[r] = sum_c x[c] * W[r][c].
// Lanes own one 32-column group; G = cols/32 lanes cooperate on a row
// (64/G rows per wave instruction when G < 64). x stays in registers.
// Optional fused final RMSNorm prologue and greedy argmax epilogue.
// ---------------------------------------------------------------------------


template <int FMT, int U>
__global__ __launch_bounds__(256) void rowdot_kernel(RowdotParams p) {
    constexpr int NT = 256;
    __shared__ float wred[NT / kWave];
    __shared__ float s_val[NT / kWave];
    __shared__ uint32_t s_idx[NT / kWave];
    __shared__ int s_last;

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t G = p.cols / 32;
    const uint32_t rpw = kWave / G;                 // rows per wave instruction
    const uint32_t g = lane % G;
    const uint32_t ro = lane / G;

    float inv_rms = 1.0f;
    if (p.gamma) {
        float ss = 0.f;
        for (uint32_t i = t; i < p.cols; i += NT) { const float v = p.x[i]; ss += v * v; }
        ss = block_sum<NT>(ss, wred);
        inv_rms = 1.0f / sqrtf(ss / (float)p.cols + 1e-6f);
    }
    float xr[32];
    float xsum = 0.f;
#pragma unroll
    for (int c = 0; c < 32; ++c) {
        const uint32_t i = g * 32 + c;
        float v = p.x[i];
        if (p.gamma) v = v * inv_rms * h2f(p.gamma[i]);
        xr[c] = v;
        xsum += v;
    }

    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    const uint32_t total_waves = gridDim.x * (NT / kWave);
    const uint32_t gw = blockIdx.x * (NT / kWave) + wave;
    const uint32_t row_step = total_waves * rpw;
    for (uint32_t rb = gw * rpw; rb < p.rows; rb += row_step * U) {
        float dots[U];
        if constexpr (FMT == FMT_Q4) {
            uint4 wv[U];
            uint16_t sv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t r = rb + u * row_step + ro;
                if (r < p.rows) {
                    wv[u] = *reinterpret_cast<const uint4*>(p.w + ((uint64_t)r * G + g) * 16u);
                    sv[u] = p.scales[(uint64_t)r * G + g];
                } else {
                    wv[u] = make_uint4(0, 0, 0, 0);
                    sv[u] = 0;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t w4[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                float d0 = 0.f, d1 = 0.f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t lo = w4[d] & 0x0F0F0F0Fu;
                    const uint32_t hi = (w4[d] >> 4) & 0x0F0F0F0Fu;
                    d0 = fmaf(xr[d * 8 + 0], ubyte_f<0>(lo), d0);
                    d1 = fmaf(xr[d * 8 + 1], ubyte_f<0>(hi), d1);
                    d0 = fmaf(xr[d * 8 + 2], ubyte_f<1>(lo), d0);
                    d1 = fmaf(xr[d * 8 + 3], ubyte_f<1>(hi), d1);
                    d0 = fmaf(xr[d * 8 + 4], ubyte_f<2>(lo), d0);
                    d1 = fmaf(xr[d * 8 + 5], ubyte_f<2>(hi), d1);
                    d0 = fmaf(xr[d * 8 + 6], ubyte_f<3>(lo), d0);
                    d1 = fmaf(xr[d * 8 + 7], ubyte_f<3>(hi), d1);
                }
                // sum_c x_c * s * (q_c - 8) = s * (sum_c x_c q_c - 8 sum_c x_c)
                dots[u] = h2f(sv[u]) * fmaf(-8.0f, xsum, d0 + d1);
            }
        } else {
            uint4 wv[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t r = rb + u * row_step + ro;
                if (r < p.rows) {
                    const uint4* src = reinterpret_cast<const uint4*>(p.w + ((uint64_t)r * G + g) * 64u);
#pragma unroll
                    for (int v = 0; v < 4; ++v) wv[u][v] = src[v];
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v) wv[u][v] = make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float d0 = 0.f, d1 = 0.f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t w4[4] = {wv[u][v].x, wv[u][v].y, wv[u][v].z, wv[u][v].w};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        d0 = fmaf(xr[v * 8 + d * 2], h2f((uint16_t)(w4[d] & 0xFFFFu)), d0);
                        d1 = fmaf(xr[v * 8 + d * 2 + 1], h2f((uint16_t)(w4[d] >> 16)), d1);
                    }
                }
                dots[u] = d0 + d1;
            }
        }
        // reduce the G lanes of each row
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v = dots[u];
            for (uint32_t off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
            const uint32_t r = rb + u * row_step + ro;
            if (g == 0 && r < p.rows) {
                p.y[r] = v;
                if (argmax_better(v, r, best_v, best_i)) { best_v = v; best_i = r; }
            }
        }
    }

    if (!p.do_argmax) return;
    // wave argmax
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best_v, off, kWave);
        const uint32_t oi = __shfl_xor(best_i, off, kWave);
        if (argmax_better(ov, oi, best_v, best_i)) { best_v = ov; best_i = oi; }
    }
    if (lane == 0) { s_val[wave] = best_v; s_idx[wave] = best_i; }
    __syncthreads();
    if (t == 0) {
        float bv = s_val[0];
        uint32_t bi = s_idx[0];
        for (int w = 1; w < NT / kWave; ++w)
            if (argmax_better(s_val[w], s_idx[w], bv, bi)) { bv = s_val[w]; bi = s_idx[w]; }
        p.part_val[blockIdx.x] = bv;
        p.part_idx[blockIdx.x] = bi;
        __threadfence();
        const uint32_t prev = __hip_atomic_fetch_add(p.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == gridDim.x - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    best_v = -INFINITY;
    best_i = 0xFFFFFFFFu;
    for (uint32_t b = t; b < gridDim.x; b += NT) {
        const float v = p.part_val[b];
        const uint32_t i = p.part_idx[b];
        if (argmax_better(v, i, best_v, best_i)) { best_v = v; best_i = i; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best_v, off, kWave);
        const uint32_t oi = __shfl_xor(best_i, off, kWave);
        if (argmax_better(ov, oi, best_v, best_i)) { best_v = ov; best_i = oi; }
    }
    __syncthreads();
    if (lane == 0) { s_val[wave] = best_v; s_idx[wave] = best_i; }
    __syncthreads();
    if (t == 0) {
        float bv = s_val[0];
        uint32_t bi = s_idx[0];
        for (int w = 1; w < NT / kWave; ++w)
            if (argmax_better(s_val[w], s_idx[w], bv, bi)) { bv = s_val[w]; bi = s_idx[w]; }
        // no candidate above -inf: the sampler returns index 0
        const int32_t tok = (bi == 0xFFFFFFFFu) ? 0 : (int32_t)bi;
        *p.token_out = tok;
        if (p.pos) {
            const int32_t ps = *p.pos;
            p.gen[ps] = tok;
            *p.pos = ps + 1;
        }
        store_u32_release(p.counter, 0u);
    }
}

}  // namespace qora
