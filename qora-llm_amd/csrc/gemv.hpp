// Batch-1 GEMV kernels for the QORA weight formats on gfx950.
//
// Projection layout (the reference's Q4Weight / F16Weight, gemv.rs:23-38):
//   Q4 : packed[k][n/2] bytes, low nibble = even column, q in [0,15],
//        value = (q - 8) * scale; scales[k][n/32] binary16.
//   F16: data[k][n] binary16.
// acc[j] += sum_i x[i] * W[i][j]  (the outer-product gemv_q4, gemv.rs:596-675).
//
// Work decomposition (split-K, no cross-workgroup synchronisation):
//   * A "group" is 32 output columns of one input row: 16 bytes of nibbles
//     plus one scale (Q4), or 64 bytes (F16). Each lane owns one group and
//     accumulates its 32 columns in registers over RPL rows, so one 128-bit
//     load feeds 32 multiply-adds, and all RPL loads are in flight at once.
//   * A workgroup (256 lanes) covers a column tile of GT groups and a slice of
//     KR = (256/GT)*RPL input rows. Lanes t = rl*GT + gi: the GT lanes of a
//     row read GT*16 contiguous bytes (128 B or 256 B row segments).
//   * The row lanes of a group are summed through LDS; each column's sum is
//     then added to a fixed-point int64 accumulator with one fire-and-forget
//     64-bit atomic. Integer addition is exact, so the result does not
//     depend on the order the K slices land in (deterministic), and no
//     fence or counter is needed: the kernel boundary publishes the sums.
//   * The prologue builds the K slice of the input in LDS: plain x, RMSNorm
//     of the fixed-point residual, silu(gate)*up of the fixed-point gate/up
//     sums, or the merge of split attention partials. Consumers therefore
//     finish the previous phase's reduction on the fly.
// Segments: up to three weight matrices are addressed as one virtual matrix
// (q|k|v concatenated by column tiles), or two matrices are paired lane by
// lane (gate|up).
// Layouts: read in the reference layout, the GT*16-byte row segments of a
// workgroup lie a full row apart (5.5 KB for 11008 columns), which the DRAM
// serves at a fraction of its streaming rate. The decode step therefore
// reads a copy in tile layout (gemv_tile_kernel): the bytes of each
// workgroup in the order its lanes load them, one contiguous block per
// workgroup and 4 KB per load step.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace qora {

// acc += v in fixed point; a contribution of 2^20 or more (or NaN) sets *flag
// instead of wrapping the accumulator.
__device__ __forceinline__ void fixed_add(long long* p, float v, int* flag) {
    const bool ok = fabsf(v) < 1048576.0f;
    fix_flag(flag, !ok);
    atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)(ok ? to_fixed(v) : 0LL));
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float silu_g = g / (1.0f + expf(-g));
    return silu_g * u;
}

// RMSNorm statistic of a fixed-point vector: 1 / sqrt(mean(x^2) + 1e-6)
// (rms_norm_f16, gemv.rs:744-753).
template <int NT>
__device__ __forceinline__ float inv_rms_fixed(const long long* xacc, uint32_t n, float* wred) {
    float ss = 0.f;
    const uint32_t last = n - 1u;
    for (uint32_t i0 = threadIdx.x; i0 < n; i0 += 4 * NT) {
        long long v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = xacc[min(i0 + u * NT, last)];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float f = from_fixed(v[u]);
            ss += (i0 + u * NT < n) ? f * f : 0.f;
        }
    }
    ss = block_sum<NT>(ss, wred);
    return 1.0f / sqrtf(ss / (float)n + 1e-6f);
}

// Attention-merge prologue (PRO_ATTN): rows [k0, k1) are dims of heads
// k0/hd .. (k1-1)/hd of the attention output; their split partials are
// merged (online-softmax merge: out = sum_s acc_s e^(m_s - m) /
// sum_s l_s e^(m_s - m), in split order) into xs[0, nrows) (zeros past k1).
// aw: LDS of kAttnMaxSplits floats per head the slice touches. Contains
// block barriers: every thread of the block calls it.
template <int NT>
__device__ __forceinline__ void attn_merge_rows(const GemvParams& p, uint32_t k0, uint32_t k1, uint32_t nrows,
                                                float* xs, float* aw) {
    const int t = threadIdx.x;
    const uint32_t hd = p.head_dim, G = p.groups;
    const uint32_t L = (uint32_t)(*p.pos) + 1u;
    const uint32_t chunk = p.attn_chunk ? p.attn_chunk : attn_chunk_for(L);
    const uint32_t s_act = min(p.attn_s_max, (L + chunk - 1) / chunk);
    const uint32_t h0 = k0 / hd;
    const uint32_t nh = (k1 - 1) / hd - h0 + 1;
    const int wave = t / kWave, lane = t & (kWave - 1);
    for (uint32_t hh = wave; hh < nh; hh += NT / kWave) {
        const uint32_t h = h0 + hh, kvh = h / G, g = h % G;
        const float* base = p.attn_part + ((uint64_t)kvh * p.attn_s_max * G + g) * (hd + 2);
        float m = -INFINITY;
        for (uint32_t s = lane; s < s_act; s += kWave) m = fmaxf(m, base[(uint64_t)s * G * (hd + 2) + hd]);
        m = wave_max(m);
        float den = 0.f;
        for (uint32_t s = lane; s < s_act; s += kWave) {
            const float* ps = base + (uint64_t)s * G * (hd + 2);
            const float w = expf(ps[hd] - m);
            aw[hh * kAttnMaxSplits + s] = w;
            den += ps[hd + 1] * w;
        }
        den = wave_sum(den);
        const float inv = 1.0f / den;
        for (uint32_t s = lane; s < s_act; s += kWave) aw[hh * kAttnMaxSplits + s] *= inv;
    }
    __syncthreads();
    for (uint32_t i = t; i < nrows; i += NT) {
        const uint32_t r = k0 + i;
        float v = 0.f;
        if (r < k1) {
            const uint32_t h = r / hd, d = r % hd, hh = h - h0;
            const float* base = p.attn_part + ((uint64_t)(h / G) * p.attn_s_max * G + (h % G)) * (hd + 2) + d;
            for (uint32_t s = 0; s < s_act; ++s) v = fmaf(base[(uint64_t)s * G * (hd + 2)], aw[hh * kAttnMaxSplits + s], v);
        }
        xs[i] = v;
    }
    __syncthreads();
}

// Which matrix and which 32-column group lane gi of column tile `tile` reads
// (shared by the GEMV kernel and the tile-layout packer, so both agree).
// Lanes past the segment get group 0 (grp_c): their columns are never written.
struct LaneSrc {
    GemvSeg sg;
    uint32_t grp;     // group within the segment (may be past the end)
    uint32_t grp_c;   // grp clamped into the segment
};

__device__ __forceinline__ LaneSrc lane_source(const GemvParams& p, uint32_t tile, int gi, int gt) {
    int sidx;
    uint32_t grp;
    if (p.paired) {
        sidx = gi < gt / 2 ? 0 : 1;
        grp = tile * (uint32_t)(gt / 2) + (uint32_t)(gi % (gt / 2));
    } else {
        sidx = 0;
        if (p.nseg > 1 && tile >= p.seg[1].tile0) sidx = 1;
        if (p.nseg > 2 && tile >= p.seg[2].tile0) sidx = 2;
        uint32_t t00 = p.seg[0].tile0, t01 = p.seg[1].tile0, t02 = p.seg[2].tile0;
        asm volatile("" : "+s"(t00), "+s"(t01), "+s"(t02));
        const uint32_t t0 = sidx == 0 ? t00 : (sidx == 1 ? t01 : t02);
        grp = (tile - t0) * (uint32_t)gt + (uint32_t)gi;
    }
    // Per-field selects over the kernarg values (a per-lane index into
    // p.seg would fetch the struct with a vector load before any weight load).
    // Each candidate is read into a scalar register first (the empty asm):
    // otherwise the compiler folds the select chain into an indexed load of
    // the argument block, which makes it copy the whole block to scratch.
    auto pick = [&](auto v0, auto v1, auto v2) {
        asm volatile("" : "+s"(v0), "+s"(v1), "+s"(v2));
        return sidx == 0 ? v0 : (sidx == 1 ? v1 : v2);
    };
    LaneSrc s;
    s.sg.w = pick(p.seg[0].w, p.seg[1].w, p.seg[2].w);
    s.sg.scales = pick(p.seg[0].scales, p.seg[1].scales, p.seg[2].scales);
    s.sg.groups = pick(p.seg[0].groups, p.seg[1].groups, p.seg[2].groups);
    s.sg.tile0 = pick(p.seg[0].tile0, p.seg[1].tile0, p.seg[2].tile0);
    s.sg.col0 = pick(p.seg[0].col0, p.seg[1].col0, p.seg[2].col0);
    s.sg.tiles = 0;
    s.grp = grp;
    s.grp_c = grp < s.sg.groups ? grp : 0u;
    return s;
}

// Tile-layout packer: one workgroup per (GEMV workgroup b, row step j)
// copies what lane t of GEMV workgroup b loads at step j (16 B of Q4 or 64 B
// of F16, and the Q4 scale) into load order. grid = blocks * rpl, 256 lanes.
template <int FMT>
__global__ __launch_bounds__(256) void gemv_tile_kernel(GemvParams p, int gt, int rpl, uint8_t* tw, uint16_t* ts) {
    const int t = threadIdx.x;
    const uint32_t b = blockIdx.x / (uint32_t)rpl;
    const uint32_t j = blockIdx.x % (uint32_t)rpl;
    const uint32_t tile = b % p.tiles, split = b / p.tiles;
    const uint32_t RL = 256u / (uint32_t)gt;
    const LaneSrc src = lane_source(p, tile, t % gt, gt);
    const uint32_t r = min(split * p.rows_per_split + (uint32_t)(t / gt) + j * RL, p.k - 1u);
    if constexpr (FMT == FMT_Q4) {
        const uint4 v = *reinterpret_cast<const uint4*>(src.sg.w + ((uint64_t)r * src.sg.groups + src.grp_c) * 16u);
        *reinterpret_cast<uint4*>(tw + (((uint64_t)b * rpl + j) * 256u + t) * 16u) = v;
        ts[((uint64_t)b * 256u + t) * rpl + j] = src.sg.scales[(uint64_t)r * src.sg.groups + src.grp_c];
    } else {
        const uint4* s = reinterpret_cast<const uint4*>(src.sg.w + ((uint64_t)r * src.sg.groups + src.grp_c) * 64u);
#pragma unroll
        for (int v = 0; v < 4; ++v)
            *reinterpret_cast<uint4*>(tw + ((((uint64_t)b * rpl + j) * 4u + v) * 256u + t) * 16u) = s[v];
    }
}

template <int FMT, int GT, int RPL, int PRO, bool TILED>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* tw, const uint16_t* ts, const void* xin,
                                                   const void* xaux, uint32_t k, uint32_t tiles_a, uint32_t rps,
                                                   uint32_t ss_nn, GemvParams p) {
    // (the arguments of the first loads come ahead of the parameter block and
    // are preloaded into scalar registers at wave launch: tile-layout
    // weights and scales, the input and its second operand, K, the tile
    // count, the rows per K slice, ss_n | norm_n << 8)
    const uint32_t ss_n = ss_nn & 0xFFu, norm_n = ss_nn >> 8;
    const long long* xacc = static_cast<const long long*>(xin);
    constexpr int NT = 256;
    constexpr int RL = NT / GT;          // row lanes
    constexpr int COLS = GT * 32;        // columns per tile
    constexpr int KR = RL * RPL;         // rows per workgroup
    constexpr int RED_STRIDE = 33;       // padded group stride in LDS
    constexpr int CPT = COLS / NT;       // columns per thread in the reduction
    constexpr int MAXH = KR / 32 + 1;    // heads a K slice can touch (head_dim >= 32)
    constexpr bool kStage = PRO == PRO_ATTN;   // only the attention merge stages x in LDS

    __shared__ float xs[kStage ? KR : 1];
    __shared__ float red[NT * RED_STRIDE];
    __shared__ float wred[NT / kWave];
    __shared__ float aw[kStage ? kAttnMaxSplits * MAXH : 1];

    const int t = threadIdx.x;
    const int gi = t % GT;
    const int rl = t / GT;
    const uint32_t tile = blockIdx.x % tiles_a;
    const uint32_t split = blockIdx.x / tiles_a;
    const uint32_t k0 = split * rps;
    const uint32_t k1 = min(k, k0 + rps);
    const uint32_t klast = k - 1u;
    // (the accumulator this launch clears is cleared at the end: stores issued
    // first would count in vmcnt ahead of the input and weight loads)

    // ---- which segment / group this lane reads ----
    const LaneSrc src = lane_source(p, tile, gi, GT);
    const GemvSeg& sg = src.sg;
    // Every load is unconditional, so all of a lane's loads are in flight
    // together and the math on row j starts when row j arrives: rows past
    // the slice read a valid row and get a zero input; lanes past the
    // segment read group 0 and their columns are never written.
    const uint32_t grp_c = src.grp_c;

    // ---- 1. input values of this lane's rows (direct loads, no LDS) ----
    float xv[RPL];
    long long xa[PRO == PRO_PLAIN || PRO == PRO_ATTN ? 1 : RPL];
    long long ua[PRO == PRO_SILU_FIXED ? RPL : 1];
    uint32_t gm[PRO == PRO_GAMMA_FIXED ? RPL : 1];
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        const uint32_t rc = min(k0 + rl + j * RL, klast);
        if constexpr (PRO == PRO_PLAIN) xv[j] = static_cast<const float*>(xin)[rc];
        if constexpr (PRO == PRO_GAMMA_FIXED) {
            xa[j] = xacc[rc];
            gm[j] = static_cast<const uint16_t*>(xaux)[rc];
        }
        if constexpr (PRO == PRO_SILU_FIXED) {
            xa[j] = xacc[rc];
            ua[j] = xacc[k + rc];
        }
    }
    float ss_part = 0.f;
    if constexpr (PRO == PRO_SILU_FIXED) ss_part = static_cast<const float*>(xaux)[min((uint32_t)(t & (kWave - 1)), ss_n - 1u)];

    // ---- 2. weight loads ----
    float acc[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[c] = 0.f;
    uint4 wq[FMT == FMT_Q4 ? RPL : 1];
    uint32_t sq[FMT == FMT_Q4 ? RPL : 1];
    if constexpr (FMT == FMT_Q4 && TILED) {
        // one contiguous block per workgroup: step j reads 4 KB, lane t 16 B
        const uint8_t* bw = tw + (uint64_t)blockIdx.x * (RPL * 4096u) + (uint32_t)t * 16u;
#pragma unroll
        for (int j = 0; j < RPL; ++j) wq[j] = *reinterpret_cast<const uint4*>(bw + j * 4096u);
        // the lane's RPL scales are adjacent
        const uint16_t* bs = ts + ((uint64_t)blockIdx.x * 256u + (uint32_t)t) * RPL;
        if constexpr (RPL >= 8) {
#pragma unroll
            for (int h = 0; h < RPL / 8; ++h) {
                const uint4 v = reinterpret_cast<const uint4*>(bs)[h];
                const uint32_t v4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sq[8 * h + 2 * e] = v4[e] & 0xFFFFu;
                    sq[8 * h + 2 * e + 1] = v4[e] >> 16;
                }
            }
        } else if constexpr (RPL == 4) {
            const uint2 v = *reinterpret_cast<const uint2*>(bs);
            sq[0] = v.x & 0xFFFFu; sq[1] = v.x >> 16; sq[2] = v.y & 0xFFFFu; sq[3] = v.y >> 16;
        } else if constexpr (RPL == 2) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(bs);
            sq[0] = v & 0xFFFFu; sq[1] = v >> 16;
        } else {
            sq[0] = bs[0];
        }
    } else if constexpr (FMT == FMT_Q4) {
        const uint64_t row_bytes = (uint64_t)sg.groups * 16u;
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const uint32_t r = min(k0 + rl + j * RL, klast);
            wq[j] = *reinterpret_cast<const uint4*>(sg.w + r * row_bytes + (uint64_t)grp_c * 16u);
            sq[j] = sg.scales[(uint64_t)r * sg.groups + grp_c];
        }
    }

    // ---- 3. the input values ----
    float ssq = 0.f;   // PRO_GAMMA_FIXED: sum of x^2 over this lane's rows
    if constexpr (PRO == PRO_GAMMA_FIXED) {
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const bool ok = k0 + rl + j * RL < k1;
            const float xf = ok ? from_fixed(xa[j]) : 0.f;
            fix_flag(p.range_flag, ok && fix_out_of_range(xa[j], kFixReadLimit));
            ssq += xf * xf;
            xv[j] = xf * h2f((uint16_t)gm[j]);
        }
    } else if constexpr (PRO == PRO_SILU_FIXED) {
        const float inv = 1.0f / sqrtf(wave_sum(t % kWave < (int)ss_n ? ss_part : 0.f) / (float)norm_n + 1e-6f);
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const bool ok = k0 + rl + j * RL < k1;
            xv[j] = ok ? silu_mul(inv * from_fixed(xa[j]), inv * from_fixed(ua[j])) : 0.f;
        }
    } else if constexpr (PRO == PRO_PLAIN) {
#pragma unroll
        for (int j = 0; j < RPL; ++j) xv[j] = (k0 + rl + j * RL < k1) ? xv[j] : 0.f;
    } else {
        attn_merge_rows<NT>(p, k0, k1, KR, xs, aw);
#pragma unroll
        for (int j = 0; j < RPL; ++j) xv[j] = xs[rl + j * RL];
    }

    if constexpr (FMT == FMT_Q4) {
        const NibbleConsts nk = nibble_consts();
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const float sx = h2f((uint16_t)sq[j]) * xv[j];
            const uint32_t w4[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const Nib8 nb = unpack_nibbles(w4[d], nk);
                acc[d * 8 + 0] = fmaf(f16lo(nb.c04), sx, acc[d * 8 + 0]);
                acc[d * 8 + 4] = fmaf(f16hi(nb.c04), sx, acc[d * 8 + 4]);
                acc[d * 8 + 1] = fmaf(f16lo(nb.c15), sx, acc[d * 8 + 1]);
                acc[d * 8 + 5] = fmaf(f16hi(nb.c15), sx, acc[d * 8 + 5]);
                acc[d * 8 + 2] = fmaf(f16lo(nb.c26), sx, acc[d * 8 + 2]);
                acc[d * 8 + 6] = fmaf(f16hi(nb.c26), sx, acc[d * 8 + 6]);
                acc[d * 8 + 3] = fmaf(f16lo(nb.c37), sx, acc[d * 8 + 3]);
                acc[d * 8 + 7] = fmaf(f16hi(nb.c37), sx, acc[d * 8 + 7]);
            }
        }
    } else {
        const uint64_t row_bytes = (uint64_t)sg.groups * 64u;
        constexpr int B = RPL < 4 ? RPL : 4;   // rows of 64 B in flight per batch
#pragma unroll
        for (int j0 = 0; j0 < RPL; j0 += B) {
            uint4 wv[B][4];
#pragma unroll
            for (int j = 0; j < B; ++j) {
                if constexpr (TILED) {
                    const uint8_t* bw = tw + ((uint64_t)blockIdx.x * RPL + (uint32_t)(j0 + j)) * 16384u +
                                        (uint32_t)t * 16u;
#pragma unroll
                    for (int v = 0; v < 4; ++v) wv[j][v] = *reinterpret_cast<const uint4*>(bw + v * 4096u);
                } else {
                    const uint32_t r = min(k0 + rl + (j0 + j) * RL, klast);
                    const uint4* wsrc = reinterpret_cast<const uint4*>(sg.w + r * row_bytes + (uint64_t)grp_c * 64u);
#pragma unroll
                    for (int v = 0; v < 4; ++v) wv[j][v] = wsrc[v];
                }
            }
#pragma unroll
            for (int j = 0; j < B; ++j) {
                const float xr = xv[j0 + j];
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

    // sum of x^2 of the K slice (each row once: the gi == 0 lanes of tile 0)
    if constexpr (PRO == PRO_GAMMA_FIXED) {
        const float ws = wave_sum((gi == 0) ? ssq : 0.f);
        if ((t & (kWave - 1)) == 0) wred[t / kWave] = ws;
    }

    // ---- reduce the RL row lanes of each group through LDS ----
    {
        float* dst = red + (rl * GT + gi) * RED_STRIDE;
#pragma unroll
        for (int c = 0; c < 32; ++c) dst[c] = acc[c];
    }
    __syncthreads();
    if constexpr (PRO == PRO_GAMMA_FIXED) {
        if (t == 0 && tile == 0) {
            float ws = 0.f;
#pragma unroll
            for (int w = 0; w < NT / kWave; ++w) ws += wred[w];
            p.ss_out[split] = ws;
        }
    }
#pragma unroll
    for (int cc = 0; cc < CPT; ++cc) {
        const int col = t + cc * NT;
        const int g = col / 32, c = col % 32;
        float s = 0.f;
#pragma unroll 8
        for (int r = 0; r < RL; ++r) s += red[(r * GT + g) * RED_STRIDE + c];
        // tile column -> (segment, local column) -> accumulator slot
        uint32_t local, lim, col0;
        if (p.paired) {
            const bool up = g >= GT / 2;
            local = tile * (COLS / 2) + (uint32_t)(col - (up ? COLS / 2 : 0));
            lim = (up ? p.seg[1].groups : p.seg[0].groups) * 32u;
            col0 = up ? p.seg[1].col0 : p.seg[0].col0;
        } else {
            local = (tile - sg.tile0) * COLS + (uint32_t)col;
            lim = sg.groups * 32u;
            col0 = sg.col0;
        }
        if (local < lim) fixed_add(p.acc + col0 + local, s, p.range_flag);
    }
    // the accumulator this launch clears (for a later kernel), after the
    // launch's own loads
    if (p.zero_ptr)
        for (uint32_t i = blockIdx.x * NT + t; i < p.zero_n; i += gridDim.x * NT) p.zero_ptr[i] = 0;
}

// acc (fixed point) -> y (fp32); paired: y[j] = silu(acc[j]) * acc[n + j].
__global__ __launch_bounds__(256) void acc_to_f32_kernel(const long long* acc, uint32_t n, int paired, float* y) {
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x)
        y[j] = paired ? silu_mul(from_fixed(acc[j]), from_fixed(acc[n + j])) : from_fixed(acc[j]);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(long long* p, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

// ---------------------------------------------------------------------------
// Row-dot GEMV over a [rows][cols] matrix (the tied lm_head,
// lm_head_parallel_q4 / _f16, gemv.rs:805-864): y[r] = sum_c x[c] * W[r][c].
// Lanes own one 32-column group; G = cols/32 lanes cooperate on a row
// (64/G rows per wave instruction when G < 64). x stays in registers.
// Optional fused final RMSNorm prologue and per-workgroup greedy argmax
// (the last step, over the workgroup bests, is argmax_finish_kernel).
// ---------------------------------------------------------------------------

template <int FMT, int U>
__global__ __launch_bounds__(256) void rowdot_kernel(RowdotParams p) {
    constexpr int NT = 256;
    __shared__ float wred[NT / kWave];
    __shared__ float s_val[NT / kWave];
    __shared__ uint32_t s_idx[NT / kWave];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t G = p.cols / 32;
    const uint32_t rpw = kWave / G;                 // rows per wave instruction
    const uint32_t g = lane % G;
    const uint32_t ro = lane / G;

    float inv_rms = 1.0f;
    if (p.gamma) {
        if (p.xacc) {
            inv_rms = inv_rms_fixed<NT>(p.xacc, p.cols, wred);
        } else {
            float ss = 0.f;
            for (uint32_t i = t; i < p.cols; i += NT) { const float v = p.x[i]; ss += v * v; }
            ss = block_sum<NT>(ss, wred);
            inv_rms = 1.0f / sqrtf(ss / (float)p.cols + 1e-6f);
        }
    }
    float xr[32];
    if (p.xacc) {
        const longlong2* src = reinterpret_cast<const longlong2*>(p.xacc + g * 32);
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const longlong2 v = src[c];
            fix_flag(p.range_flag, fix_out_of_range(v.x, kFixReadLimit) || fix_out_of_range(v.y, kFixReadLimit));
            xr[2 * c] = from_fixed(v.x);
            xr[2 * c + 1] = from_fixed(v.y);
        }
    } else {
        const float4* src = reinterpret_cast<const float4*>(p.x + g * 32);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 v = src[c];
            xr[4 * c] = v.x;
            xr[4 * c + 1] = v.y;
            xr[4 * c + 2] = v.z;
            xr[4 * c + 3] = v.w;
        }
    }
    if (p.gamma) {
        const uint4* gsrc = reinterpret_cast<const uint4*>(p.gamma + g * 32);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 gv = gsrc[c];
            const uint32_t w4[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                xr[c * 8 + 2 * d] = xr[c * 8 + 2 * d] * inv_rms * h2f((uint16_t)(w4[d] & 0xFFFFu));
                xr[c * 8 + 2 * d + 1] = xr[c * 8 + 2 * d + 1] * inv_rms * h2f((uint16_t)(w4[d] >> 16));
            }
        }
    }
    const NibbleConsts nk = nibble_consts();

    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    const uint32_t total_waves = gridDim.x * (NT / kWave);
    const uint32_t gw = blockIdx.x * (NT / kWave) + wave;
    const uint32_t row_step = total_waves * rpw;
    for (uint32_t rb = gw * rpw; rb < p.rows; rb += row_step * U) {
        float dots[U];
        if constexpr (FMT == FMT_Q4) {
            uint4 wv[U];
            uint32_t sv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t r = min(rb + u * row_step + ro, p.rows - 1u);
                wv[u] = *reinterpret_cast<const uint4*>(p.w + ((uint64_t)r * G + g) * 16u);
                sv[u] = p.scales[(uint64_t)r * G + g];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t w4[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                float d0 = 0.f, d1 = 0.f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const Nib8 nb = unpack_nibbles(w4[d], nk);
                    d0 = fmaf(f16lo(nb.c04), xr[d * 8 + 0], d0);
                    d1 = fmaf(f16hi(nb.c04), xr[d * 8 + 4], d1);
                    d0 = fmaf(f16lo(nb.c15), xr[d * 8 + 1], d0);
                    d1 = fmaf(f16hi(nb.c15), xr[d * 8 + 5], d1);
                    d0 = fmaf(f16lo(nb.c26), xr[d * 8 + 2], d0);
                    d1 = fmaf(f16hi(nb.c26), xr[d * 8 + 6], d1);
                    d0 = fmaf(f16lo(nb.c37), xr[d * 8 + 3], d0);
                    d1 = fmaf(f16hi(nb.c37), xr[d * 8 + 7], d1);
                }
                // sum_c x_c * s * (q_c - 8) = s * sum_c x_c * (q_c - 8)
                dots[u] = h2f(sv[u]) * (d0 + d1);
            }
        } else {
            uint4 wv[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t r = min(rb + u * row_step + ro, p.rows - 1u);
                const uint4* src = reinterpret_cast<const uint4*>(p.w + ((uint64_t)r * G + g) * 64u);
#pragma unroll
                for (int v = 0; v < 4; ++v) wv[u][v] = src[v];
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
    }
}

// Greedy token from the per-workgroup bests (generate.rs:346-352): one block.
__global__ __launch_bounds__(256) void argmax_finish_kernel(ArgmaxFinishParams p) {
    __shared__ float s_val[4];
    __shared__ uint32_t s_idx[4];
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t b = threadIdx.x; b < p.parts; b += 256) {
        const float v = p.part_val[b];
        const uint32_t i = p.part_idx[b];
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
        // no candidate above -inf: the sampler returns index 0
        const int32_t tok = (i0 == 0xFFFFFFFFu) ? 0 : (int32_t)i0;
        *p.token_out = tok;
        if (p.pos) {
            const int32_t ps = *p.pos;
            p.gen[ps] = tok;
            *p.pos = ps + 1;
        }
        if (p.host_token) {
            // the range flag of the step's fixed-point values, then the token
            // last, after the step's other stores are visible: a host that
            // reads the token without waiting for the kernel's end finds
            // every result of the step in place
            if (p.range_flag) p.host_token[1] = *p.range_flag;
            __threadfence_system();
            *p.host_token = tok;
        }
    }
}

}  // namespace qora
