// Q4 GEMV on the gfx950 integer matrix cores (v_mfma_i32_16x16x64_i8).
//
// y[j] = sum_k x[k] * s[k][g(j)] * (q[k][j] - 8)   (gemv_q4, gemv.rs:596-675)
//
// At batch 1 a VALU GEMV spends ~2 instructions per nibble (unpack, convert,
// multiply-add) and is bound by issue, not by HBM. Here the multiply-add
// runs on the matrix cores in exact integer arithmetic:
//   * weights: the int8 B operand is 16 * (q - 8), made from packed nibbles
//     by one bit operation per 4 nibbles: (w & 0xF0F0F0F0) ^ 0x80808080 maps
//     a high nibble q to the byte 16q - 128 = 16 (q - 8) (two's complement),
//     and the low nibbles take the same after a 4-bit shift;
//   * inputs: z[k][g] = x[k] * s[k][g] (fp32) is quantised against a block
//     exponent E (2^E bounds |z| over the K slice of the group) to the
//     integer M = round(z * 2^(30-E)), |M| <= 2^30, split into four signed
//     base-256 digits ("limbs", each in [-128, 127]: M + 0x808080 with the
//     low three bytes re-centred by ^ 0x80), which form rows 0..3 of the A
//     operand (rows 4..15 are zero);
//   * the MFMA sums limb * 16 (q - 8) over 64 rows in int32 (|C| < 2^22 per
//     slice), and C0 + 2^8 C1 + 2^16 C2 + 2^24 C3 = sum_k M_k * 16 (q_k - 8)
//     exactly; times 2^(E-34) it is the slice's contribution, which lands in
//     the fixed-point accumulator (value * 2^36) as one int64 atomic.
// Every step after the fp32 product x*s is exact, so the result is
// deterministic, and the only rounding (|M| quantised to 2^-30 of the
// block bound) is ~2^-27 of the largest term, below fp32 accumulation error.
//
// Operand layouts of v_mfma_i32_16x16x64_i8 (lane l, byte b = 0..15):
//   A[i = l % 16][k = 16 (l / 16) + b], B[k = 16 (l / 16) + b][j = l % 16],
//   C[i = 4 (l / 16) + r][j = l % 16] in result register r.
// So lanes 0..15 end with the four limb sums of column j = l.
//
// Work decomposition: a workgroup is 4 waves x GW groups (32 columns each)
// over a K slice of KW rows (a multiple of 64); all 4 waves share the slice.
// Column tiles map to (segment, group) through lane_source with
// gt = 4 * GW, so q|k|v concatenation and gate|up pairing work as in the
// VALU kernel. Tile layout (gemv_q4m_pack_kernel), per (workgroup, wave):
//   tw: [group g < GW][K block kb < KW/64][lane < 64] x 16 B: lane l's B
//       fragments of column blocks 2g (bytes 0-7) and 2g+1 (bytes 8-15) for
//       column 16 * blk + l % 16 and rows 64 kb + 16 (l / 16) + b; in each
//       8-byte fragment, byte m of word w holds row 8w + m in its high
//       nibble and row 8w + 4 + m in its low nibble;
//   ts: [lane][u < NZ] scales of the lane's z values (e = lane * NZ + u:
//       row e % KW, group e / KW);
//   tes: [group] exponent bound of the slice's scales (max |s| <= 2^tes).
#pragma once

#include "common.hpp"
#include "gemv.hpp"
#include "params.hpp"

namespace qora {

typedef int v4i32 __attribute__((ext_vector_type(4)));

// exponent bound of a binary16 magnitude: |s| <= 2^e
__device__ __forceinline__ int f16_exp_bound(uint16_t h) {
    const int e = (h >> 10) & 0x1F;
    return e == 0 ? -14 : e - 14;
}

// One workgroup per (GEMV workgroup b, wave w), 64 lanes: lane l writes its
// 16-byte fragment pair for every (group, K block), its NZ scales, and lanes
// 0..gw-1 the exponent bound of their group.
__global__ __launch_bounds__(64) void gemv_q4m_pack_kernel(GemvParams p, int gw, int kw, uint8_t* tw, uint16_t* ts,
                                                           int8_t* te) {
    const uint32_t l = threadIdx.x;
    const uint32_t b = blockIdx.x / 4, w = blockIdx.x % 4;
    const uint32_t tile = b % p.tiles, split = b / p.tiles;
    const uint32_t k0 = split * (uint32_t)kw;
    const uint32_t k1 = min(p.k, k0 + (uint32_t)kw);
    const uint32_t nkb = (uint32_t)kw / 64, nz = (uint32_t)(gw * kw) / 64;
    const uint64_t bw = (uint64_t)b * 4 + w;
    for (int g = 0; g < gw; ++g) {
        const LaneSrc src = lane_source(p, tile, (int)w * gw + g, 4 * gw);
        const uint64_t row_bytes = (uint64_t)src.sg.groups * 16u;
        for (uint32_t kb = 0; kb < nkb; ++kb) {
            uint32_t word[4];
            for (int half = 0; half < 2; ++half) {
                const uint32_t c = src.grp_c * 32u + (uint32_t)half * 16u + (l % 16);   // column in the segment
                const uint32_t rbase = k0 + kb * 64u + 16u * (l / 16);
                for (int wi = 0; wi < 2; ++wi) {
                    uint32_t v = 0;
                    for (int m = 0; m < 4; ++m) {
                        const uint32_t rh = min(rbase + 8u * wi + m, p.k - 1u);
                        const uint32_t rl = min(rbase + 8u * wi + 4u + m, p.k - 1u);
                        const uint8_t bh = src.sg.w[rh * row_bytes + c / 2];
                        const uint8_t bl = src.sg.w[rl * row_bytes + c / 2];
                        const uint32_t qh = (c & 1) ? (bh >> 4) : (bh & 0xF);
                        const uint32_t ql = (c & 1) ? (bl >> 4) : (bl & 0xF);
                        v |= ((qh << 4) | ql) << (8 * m);
                    }
                    word[half * 2 + wi] = v;
                }
            }
            *reinterpret_cast<uint4*>(tw + ((bw * gw + g) * nkb + kb) * 1024u + l * 16u) =
                make_uint4(word[0], word[1], word[2], word[3]);
        }
    }
    for (uint32_t u = 0; u < nz; ++u) {
        const uint32_t e = l * nz + u;
        const LaneSrc src = lane_source(p, tile, (int)(w * gw + e / (uint32_t)kw), 4 * gw);
        const uint32_t r = min(k0 + e % (uint32_t)kw, p.k - 1u);
        ts[(bw * 64u + l) * nz + u] = src.sg.scales[(uint64_t)r * src.sg.groups + src.grp_c];
    }
    if (l < (uint32_t)gw) {
        const LaneSrc src = lane_source(p, tile, (int)(w * gw + l), 4 * gw);
        int eb = -14;
        for (uint32_t r = k0; r < k1; ++r)
            eb = max(eb, f16_exp_bound(src.sg.scales[(uint64_t)r * src.sg.groups + src.grp_c] & 0x7FFFu));
        te[bw * gw + l] = (int8_t)eb;
    }
}

// 16 nibbles (8 bytes) -> B fragment of 16 int8 values 16 * (q - 8)
__device__ __forceinline__ v4i32 q4_bfrag(uint32_t w0, uint32_t w1) {
    v4i32 r;
    r[0] = (int)((w0 & 0xF0F0F0F0u) ^ 0x80808080u);
    r[1] = (int)(((w0 << 4) & 0xF0F0F0F0u) ^ 0x80808080u);
    r[2] = (int)((w1 & 0xF0F0F0F0u) ^ 0x80808080u);
    r[3] = (int)(((w1 << 4) & 0xF0F0F0F0u) ^ 0x80808080u);
    return r;
}

// Weight fragments of one wave: [group][K block] x 16 B per lane.
template <int GW, int NKB>
__device__ __forceinline__ void gemv_q4m_load_weights(const uint8_t* tw, uint64_t bw, int lane, uint4 (&wq)[GW][NKB]) {
    const uint8_t* src = tw + bw * (uint64_t)(GW * NKB * 1024) + (uint32_t)lane * 16u;
#pragma unroll
    for (int g = 0; g < GW; ++g)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) wq[g][kb] = ld_stream(src + (g * NKB + kb) * 1024);
}

// The lane's NZ scales (adjacent binary16) and the wave's exponent bounds.
// The bounds stay per-lane values (every lane loads the same byte) until the
// quantisation reads them: taking them to a scalar here would wait for the
// load before the weight loads are issued.
template <int GW, int NZ>
__device__ __forceinline__ void gemv_q4m_load_scales(const uint16_t* ts, const int8_t* tes, uint64_t bw, int lane,
                                                     uint32_t (&sw)[(NZ + 1) / 2], int (&esg)[GW]) {
    const uint16_t* src = ts + (bw * 64u + (uint32_t)lane) * NZ;
    if constexpr (NZ >= 8) {
#pragma unroll
        for (int h = 0; h < NZ / 8; ++h) {
            const uint4 v = ld_stream(reinterpret_cast<const uint4*>(src) + h);
            sw[4 * h] = v.x;
            sw[4 * h + 1] = v.y;
            sw[4 * h + 2] = v.z;
            sw[4 * h + 3] = v.w;
        }
    } else if constexpr (NZ == 4) {
        const uint2 v = ld_stream2(src);
        sw[0] = v.x;
        sw[1] = v.y;
    } else if constexpr (NZ == 2) {
        sw[0] = *reinterpret_cast<const uint32_t*>(src);
    } else {
        sw[0] = src[0];
    }
#pragma unroll
    for (int g = 0; g < GW; ++g) esg[g] = (int)tes[bw * GW + g];
}


// Attention-merge prologue run by one wave (see attn_merge_rows) for rows
// [r0, r1) of the slice that starts at k0 (r1 - r0 <= 32, so at most two
// heads): the per-split weights of each head the rows touch, then each row's
// merge, with lane l taking row r0 + l % 32 and the splits of parity l / 32.
// Slots past the active splits are skipped by selection, so stale bits never
// reach the sum. aw: LDS of kAttnMaxSplits floats per head, private to the
// calling wave.
// Latency: every load is issued with the position load, before the number
// of active splits is known: the running max and sum of every split (lane s:
// split s) and the row of every split up to the launch's split count (slots
// past the active splits are read but never selected).

// The arguments gemv_q4m_kernel's first loads need, preloaded into scalar
// registers at wave launch (leading kernel arguments); the rest comes from
// the GemvParams block.
struct GemvFirst {
    const uint8_t* tw;
    const uint16_t* ts;
    const int8_t* tes;
    const float* attn_part;
    const int32_t* pos;
    uint32_t k, tiles, hd, groups, s_max;
};

__device__ __forceinline__ void attn_merge_rows_wave(const GemvParams& p, const GemvFirst& f, uint32_t k0, uint32_t r0,
                                                     uint32_t r1, uint32_t k1, float* xs, float* aw) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t hd = f.hd, G = f.groups, s_max = f.s_max;
    const uint64_t sstride = (uint64_t)G * (hd + 2);
    const uint32_t a0 = k0 + r0, a1 = min(k0 + r1, k1);      // absolute rows
    if (a0 >= a1) {
        for (uint32_t i = r0 + (uint32_t)lane; i < r1; i += kWave) xs[i] = 0.f;
        return;
    }
    const uint32_t h0 = a0 / hd;
    const uint32_t nh = (a1 - 1) / hd - h0 + 1;                // 1 or 2
    const uint32_t i = r0 + (uint32_t)(lane % 32);
    const uint32_t par = (uint32_t)lane / 32;
    const uint32_t r = min(k0 + i, a1 - 1u);
    const uint32_t h = r / hd, d = r % hd, hh = h - h0;
    const float* rbase = f.attn_part + ((uint64_t)(h / G) * s_max * G + (h % G)) * (hd + 2) + d;
    // ---- issued together: position, every split's (m, l), the first rows ----
    const int32_t pos_raw = *f.pos;
    const uint32_t sl = min((uint32_t)lane, s_max - 1u);
    float ms[2], ls[2];
#pragma unroll
    for (uint32_t q = 0; q < 2; ++q) {
        const uint32_t hq = h0 + min(q, nh - 1u);
        const float* base = f.attn_part + ((uint64_t)(hq / G) * s_max * G + hq % G) * (hd + 2);
        ms[q] = base[(uint64_t)sl * sstride + hd];
        ls[q] = base[(uint64_t)sl * sstride + hd + 1];
    }
    float pv[kAttnMaxSplits / 2];
#pragma unroll
    for (uint32_t j = 0; j < kAttnMaxSplits / 2; ++j)
        pv[j] = rbase[(uint64_t)min(par + 2u * j, s_max - 1u) * sstride];
    const uint32_t L = (uint32_t)pos_raw + 1u;
    const uint32_t chunk = p.attn_chunk ? p.attn_chunk : attn_chunk_for(L);
    const uint32_t s_act = min(s_max, (L + chunk - 1) / chunk);
    const bool ok = (uint32_t)lane < s_act;
#pragma unroll
    for (uint32_t q = 0; q < 2; ++q) {
        if (q < nh) {
            const float m = wave_max(ok ? ms[q] : -INFINITY);
            const float w = ok ? expf(ms[q] - m) : 0.f;
            const float den = wave_sum(ok ? ls[q] * w : 0.f);
            aw[q * kAttnMaxSplits + lane] = w / den;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float* wrow = aw + hh * kAttnMaxSplits;
    // every weight is read unconditionally (sj < kAttnMaxSplits), so the
    // reads go out together and the inactive splits are a select: a read
    // under the condition became a branch and an LDS round trip per split
    float wj[kAttnMaxSplits / 2];
#pragma unroll
    for (uint32_t j = 0; j < kAttnMaxSplits / 2; ++j) wj[j] = wrow[par + 2u * j];
    float v = 0.f;
#pragma unroll
    for (uint32_t j = 0; j < kAttnMaxSplits / 2; ++j) {
        const uint32_t sj = par + 2u * j;
        const float t = fmaf(pv[j], wj[j], v);
        v = sj < s_act ? t : v;
    }
    v += __shfl_xor(v, 32, kWave);
    if (lane < 32 && i < r1) xs[i] = k0 + i < k1 ? v : 0.f;
}

// The item of workgroup b of a G-workgroup launch in XCD order. Workgroups
// go to the 8 XCDs in turn (b to XCD (b + r) mod 8, r fixed for the launch),
// so XCD x holds the workgroups b = x mod 8; they take the contiguous items
// [x q + min(x, G mod 8), ...) with q = G / 8, and the K slices whose inputs
// an XCD's L2 fetches are a few instead of all of them. A permutation of
// [0, G) for every G.
__device__ __forceinline__ uint32_t xcd_item(uint32_t b, uint32_t G) {
    const uint32_t q = G >> 3, rem = G & 7u, x = b & 7u;
    return x * q + min(x, rem) + (b >> 3);
}

// Where a matrix-core wave's outputs go: per group, the accumulator of its
// first column (nullptr for a group past its segment), and the range flag.
// Computed when the wave starts and held in scalar registers: read at the
// epilogue, after the weights have streamed through the caches, the kernel
// arguments would cost a chain of dependent scalar-memory round trips.
template <int GW>
struct GemvOut {
    long long* dst[GW];
    int* flag;
};

template <int GW>
__device__ __forceinline__ GemvOut<GW> gemv_q4m_out(const GemvParams& p, uint32_t tile, int wave) {
    GemvOut<GW> o;
#pragma unroll
    for (int g = 0; g < GW; ++g) {
        const LaneSrc src = lane_source(p, tile, wave * GW + g, 4 * GW);
        o.dst[g] = sgpr_ptr(src.grp < src.sg.groups ? p.acc + src.sg.col0 + src.grp * 32u : nullptr);
    }
    o.flag = sgpr_ptr(p.range_flag);
    return o;
}

// One work item (column tile, K slice) of one matrix-core wave, once the
// slice's input x is known: x * s quantised to 30-bit limbs (LDS), the
// matrix-core pass over the wave's weight fragments, and the fixed-point
// epilogue (one int64 atomic per column). xm = max |x| over the slice;
// xval(u, r) returns x of slice row r, the lane's u-th z value (r = (lane *
// NZ + u) % KW).
template <int GW, int KW, typename XVal>
__device__ __forceinline__ void gemv_q4m_item(const GemvOut<GW>& out, int lane, XVal xval, float xm,
                                              const uint32_t (&sw)[(GW * KW / 64 + 1) / 2],
                                              const int (&esv)[GW], const uint4 (&wq)[GW][KW / 64],
                                              uint8_t (*zlw)[4][KW], const uint8_t* zero16) {
    constexpr int NKB = KW / 64;
    constexpr int NZ = GW * KW / 64;
    const uint32_t li = (uint32_t)lane % 16, lk = (uint32_t)lane / 16;
    int esg[GW];
#pragma unroll
    for (int g = 0; g < GW; ++g) esg[g] = __builtin_amdgcn_readfirstlane(esv[g]);
    // 2^ex bounds max |x| (0 for an all-zero slice)
    const int ex =
        __builtin_amdgcn_readfirstlane(xm > 0.f ? (int)((__float_as_uint(xm) >> 23) & 0xFFu) - 126 : 0);

    // ---- z = x * s quantised to 30-bit integers, stored as limb bytes ----
#pragma unroll
    for (int u = 0; u < NZ; ++u) {
        const uint32_t e = (uint32_t)lane * NZ + u;
        const uint32_t rz = e % KW, gz = e / KW;
        int es = esg[0];
#pragma unroll
        for (int g = 1; g < GW; ++g) es = gz == (uint32_t)g ? esg[g] : es;
        const uint16_t sbits = (uint16_t)((u & 1) ? (sw[u / 2] >> 16) : (sw[u / 2] & 0xFFFFu));
        const float z = xval(u, rz) * h2f(sbits);
        const int M = (int)rintf(ldexpf(z, 30 - (ex + es)));
        const uint32_t limbs = (uint32_t)(M + 0x808080) ^ 0x808080u;
        uint8_t* zp = &zlw[gz][0][rz];
        zp[0] = (uint8_t)(limbs & 0xFFu);
        zp[KW] = (uint8_t)((limbs >> 8) & 0xFFu);
        zp[2 * KW] = (uint8_t)((limbs >> 16) & 0xFFu);
        zp[3 * KW] = (uint8_t)(limbs >> 24);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- matrix cores: C[limb][column] += A[limb][k] * B[k][column] ----
    v4i32 acc[2 * GW];
#pragma unroll
    for (int c = 0; c < 2 * GW; ++c) acc[c] = (v4i32){0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < GW; ++g) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const uint8_t* ap = li < 4 ? &zlw[g][li][kb * 64 + 16 * lk] : zero16;
            const v4i32 a = *reinterpret_cast<const v4i32*>(ap);
            const uint4 w = wq[g][kb];
            acc[2 * g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, q4_bfrag(w.x, w.y), acc[2 * g], 0, 0, 0);
            acc[2 * g + 1] =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(a, q4_bfrag(w.z, w.w), acc[2 * g + 1], 0, 0, 0);
        }
    }
    // the next item rewrites zl: this item's operand reads come first
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- epilogue: lanes 0..15 hold limbs 0..3 of column l of each block ----
    // Y = C0 + 2^8 C1 + 2^16 C2 + 2^24 C3 as (C0 + 2^8 C1) + 2^16 (C2 + 2^8 C3):
    // each half fits int32 (|C| < 2^22). value = Y * 2^(E - 34), so the
    // fixed-point amount (2^36 units) is Y << (E + 2), rounded when E + 2 < 0.
    if (lane < 16) {
#pragma unroll
        for (int g = 0; g < GW; ++g) {
            if (!out.dst[g]) continue;
            const int sh = max(min(ex + esg[g] + 2, 62), -62);
            const int rsh = sh < 0 ? -sh : 0, lsh = sh > 0 ? sh : 0;
            const long long rnd = rsh > 0 ? (1LL << (rsh - 1)) : 0;
            long long* dst = out.dst[g] + (uint32_t)lane;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const v4i32 c = acc[2 * g + h];
                // |C| < 2^22 for 256 rows: each half fits int32; 512 rows need 64 bits
                long long lo, hi;
                if constexpr (KW <= 256) {
                    lo = c[0] + (c[1] << 8);
                    hi = c[2] + (c[3] << 8);
                } else {
                    lo = (long long)c[0] + ((long long)c[1] << 8);
                    hi = (long long)c[2] + ((long long)c[3] << 8);
                }
                const long long Y = lo + (hi << 16);
                // contributions of 2^20 or more flag the range instead of wrapping
                const long long ay = Y < 0 ? -Y : Y;
                const bool big = lsh >= 56 ? ay != 0 : ((ay + rnd) >> rsh) >= (kFixAddLimit >> lsh);
                fix_flag(out.flag, big);
                const long long f = big ? 0 : ((Y + rnd) >> rsh) << lsh;
                atomicAdd(reinterpret_cast<unsigned long long*>(dst + h * 16), (unsigned long long)f);
            }
        }
    }
}

// Four matrix-core waves plus one prologue wave. A wave waits on its loads
// in issue order, so the roles are split by wave: the prologue wave loads
// the slice's inputs and builds x (xs in LDS) while the matrix-core waves
// stream their scales and weights from the first cycle; the one block
// barrier hands x over without waiting for the weight loads.
// IPW > 1: workgroup b of a grid of G takes the work items (column tile,
// K slice) b, b + G, ... (at most IPW), with every item's scales and weights
// requested up front. With G = the workgroups a device holds at once, the
// items past G go to the first workgroups instead of a second round that
// could only start when the first round ends.
// LDS of one gemv_q4m workgroup.
template <int GW, int KW, int PRO, int IPW>
struct GemvQ4mSmem {
    static constexpr int NPW = PRO == PRO_ATTN ? 4 : 1;
    static constexpr int MAXH = KW / 32 + 1;
    __align__(16) float xs[IPW][KW];
    float wred[IPW][2][NPW];
    __align__(16) uint8_t zl[4][GW][4][KW];   // limb bytes: [wave][group][limb][row]
    __align__(16) uint8_t zero16[16];         // A rows 4..15
    float aw[PRO == PRO_ATTN ? NPW * kAttnMaxSplits * MAXH : 1];
};

// The body of gemv_q4m_kernel for workgroup `block` of `nblocks`.
template <int GW, int KW, int PRO, int IPW>
__device__ __forceinline__ void gemv_q4m_body(const GemvParams& p, const GemvFirst& f, uint32_t block,
                                              uint32_t nblocks, GemvQ4mSmem<GW, KW, PRO, IPW>& sm) {
    constexpr int NW = 4;                    // matrix-core waves
    constexpr int NPW = PRO == PRO_ATTN ? 4 : 1;   // prologue waves (the attention merge gets four)
    constexpr int NKB = KW / 64;            // K blocks (one MFMA each) per slice
    constexpr int NZ = GW * KW / 64;        // z values per lane
    constexpr int RPW = KW / 64;            // prologue rows per lane
    constexpr int MAXH = KW / 32 + 1;       // heads a slice can touch (head_dim >= 32)
    constexpr bool kAttn = PRO == PRO_ATTN;
    static_assert(KW % 64 == 0 && KW <= 512, "slice of 64..512 rows");
    static_assert(IPW == 1 || !kAttn, "the attention-merge prologue takes one item per workgroup");
    auto& xs = sm.xs;
    auto& wred = sm.wred;
    auto& zl = sm.zl;
    auto& zero16 = sm.zero16;
    float* aw = sm.aw;

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    // wave-uniform (scalar) so segment lookups and addresses stay on the SALU
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    uint32_t tiles = __builtin_amdgcn_readfirstlane(f.tiles);
    sgpr_pin(tiles);
    // items block, block + nblocks, ... (strided, so a grid of resident
    // workgroups spreads the items beyond it over the first workgroups); one
    // item per workgroup: the grid is the item count
    uint32_t nit = 1u;
    if constexpr (IPW > 1) {
        const uint32_t items = tiles * p.splits;
        nit = block < items ? min((uint32_t)IPW, (items - block + nblocks - 1) / nblocks) : 0u;
    }

    uint4 wq[IPW][GW][NKB];
    uint32_t sw[IPW][(NZ + 1) / 2];
    int esg[IPW][GW];
    GemvOut<GW> out[IPW];
    float* ss_dst = nullptr;
    if (wave >= NW) {
        // ---- prologue wave(s): rows [k0, k1) of the input into xs, max |x|, sum x^2 ----
        // Raised issue priority: their few input loads enter the CU's memory
        // queue ahead of the weight streams of the other waves on the CU.
        __builtin_amdgcn_s_setprio(3);
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            if ((uint32_t)j >= nit) continue;
            const uint32_t split = (block + (uint32_t)j * nblocks) / tiles;
            const uint32_t k0 = split * (uint32_t)KW;
            const uint32_t k1 = min(f.k, k0 + (uint32_t)KW);
            float mx = 0.f, ss = 0.f;
            if constexpr (kAttn) {
                const uint32_t pw = (uint32_t)(wave - NW);
                constexpr uint32_t RW = KW / NPW;   // rows per prologue wave (<= 64)
#pragma unroll
                for (uint32_t c = 0; c < RW; c += 32)
                    attn_merge_rows_wave(p, f, k0, pw * RW + c, pw * RW + min(c + 32, RW), k1, xs[j],
                                         aw + pw * kAttnMaxSplits * MAXH);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                for (uint32_t i = (uint32_t)lane; i < RW; i += kWave) mx = fmaxf(mx, fabsf(xs[j][pw * RW + i]));
            } else {
                float xp[RPW], ssp = 0.f;
                long long xa[RPW], xb[RPW];
                uint16_t gm[RPW];
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const uint32_t rc = min(k0 + (uint32_t)(lane + 64 * r), f.k - 1u);
                    if constexpr (PRO == PRO_PLAIN) xp[r] = p.x[rc];
                    if constexpr (PRO == PRO_GAMMA_FIXED) {
                        xa[r] = p.xacc[rc];
                        gm[r] = p.gamma[rc];
                    }
                    if constexpr (PRO == PRO_SILU_FIXED) {
                        xa[r] = p.xacc[rc];
                        xb[r] = p.xacc[p.k + rc];
                    }
                }
                if constexpr (PRO == PRO_SILU_FIXED) {
                    const float* sp = p.ss_in + min((uint32_t)lane, p.ss_n - 1u);
                    ssp = *sp;
                }
                float inv = 1.f;
                if constexpr (PRO == PRO_SILU_FIXED)
                    inv = 1.0f / sqrtf(wave_sum(lane < (int)p.ss_n ? ssp : 0.f) / (float)p.norm_n + 1e-6f);
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const bool ok = k0 + (uint32_t)(lane + 64 * r) < k1;
                    float x;
                    if constexpr (PRO == PRO_PLAIN) {
                        x = ok ? xp[r] : 0.f;
                    } else if constexpr (PRO == PRO_GAMMA_FIXED) {
                        const float xf = ok ? from_fixed(xa[r]) : 0.f;
                        fix_flag(p.range_flag, ok && fix_out_of_range(xa[r], kFixReadLimit));
                        ss += xf * xf;
                        x = xf * h2f(gm[r]);
                    } else {
                        x = ok ? silu_mul(inv * from_fixed(xa[r]), inv * from_fixed(xb[r])) : 0.f;
                    }
                    xs[j][lane + 64 * r] = x;
                    mx = fmaxf(mx, fabsf(x));
                }
            }
            mx = wave_max(mx);
            if constexpr (PRO == PRO_GAMMA_FIXED) ss = wave_sum(ss);
            if (lane == 0) {
                wred[j][0][wave - NW] = mx;
                wred[j][1][wave - NW] = ss;
            }
        }
        if (wave == NW && lane < 4) reinterpret_cast<uint32_t*>(zero16)[lane] = 0u;
    } else {
        // ---- matrix-core waves: every item's scales first (the quantisation needs them), then weights ----
#pragma unroll
        for (int j = 0; j < IPW; ++j)
            if ((uint32_t)j < nit) gemv_q4m_load_scales<GW, NZ>(f.ts, f.tes, (uint64_t)(block + (uint32_t)j * nblocks) * NW + wave, lane, sw[j], esg[j]);
#pragma unroll
        for (int j = 0; j < IPW; ++j)
            if ((uint32_t)j < nit) gemv_q4m_load_weights<GW, NKB>(f.tw, (uint64_t)(block + (uint32_t)j * nblocks) * NW + wave, lane, wq[j]);
#pragma unroll
        for (int j = 0; j < IPW; ++j) out[j] = gemv_q4m_out<GW>(p, (block + (uint32_t)j * nblocks) % tiles, wave);
        if constexpr (PRO == PRO_GAMMA_FIXED) {
            ss_dst = sgpr_ptr(p.ss_out);
        }
    }
    __syncthreads();
    if (wave >= NW) {
        // the accumulator this launch clears, by the prologue waves once
        // their input is handed over
        if (p.zero_ptr) {
            const uint32_t tq = (uint32_t)(t - NW * kWave), nq = NPW * kWave;
            for (uint32_t i = block * nq + tq; i < p.zero_n; i += nblocks * nq) p.zero_ptr[i] = 0;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        if ((uint32_t)j >= nit) continue;
        const uint32_t item = (block + (uint32_t)j * nblocks);
        const uint32_t tile = item % tiles;
        const uint32_t split = item / tiles;
        float xm = wred[j][0][0];
#pragma unroll
        for (int w = 1; w < NPW; ++w) xm = fmaxf(xm, wred[j][0][w]);
        if constexpr (PRO == PRO_GAMMA_FIXED) {
            if (t == 0 && tile == 0)
                __hip_atomic_store(ss_dst + split, wred[j][1][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const float* xj = xs[j];
        gemv_q4m_item<GW, KW>(out[j], lane, [xj](int, uint32_t r) { return xj[r]; }, xm, sw[j], esg[j], wq[j],
                              zl[wave], zero16);
    }
}

// Arguments: what the first loads need comes first and is preloaded into
// scalar registers at wave launch (14 words): weights, scales, exponent
// bounds, the attention partials and the position, K, the tile count, the
// item count with the XCD-order flag in bit 31, and head_dim | groups << 10 |
// s_max << 20; the rest comes from the GemvParams block, read where it is
// used (no kernarg_warm, whose wait would come before the first loads).
template <int GW, int KW, int PRO, int IPW = 1>
__global__ __launch_bounds__(PRO == PRO_ATTN ? 512 : 320) void gemv_q4m_kernel(
    const uint8_t* tw, const uint16_t* ts, const int8_t* tes, const float* attn_part, const int32_t* pos, uint32_t k,
    uint32_t tiles, uint32_t items_x, uint32_t hgs, GemvParams p) {
    __shared__ GemvQ4mSmem<GW, KW, PRO, IPW> sm;
    const GemvFirst f{tw, ts, tes, attn_part, pos, k, tiles, hgs & 0x3FFu, (hgs >> 10) & 0x3FFu, hgs >> 20};
    const uint32_t n = items_x & 0x7FFFFFFFu;
    const uint32_t b = IPW == 1 ? blockIdx.x + (items_x >> 31) * (xcd_item(blockIdx.x, n) - blockIdx.x) : blockIdx.x;
    gemv_q4m_body<GW, KW, PRO, IPW>(p, f, b, IPW == 1 ? n : gridDim.x, sm);
}

// Four matrix-core waves and no prologue wave (PRO_PLAIN, PRO_GAMMA_FIXED,
// PRO_SILU_FIXED). Each wave builds a quarter of the slice's input itself:
// its input loads go out first, then its scales and weights, and loads
// complete in issue order, so the input is in long before the weights (a
// separate prologue wave's input loads would queue behind the other waves'
// weight streams). A CU holds eight such 4-wave workgroups at once against
// five 5-wave ones, so the gate|up projection's 1376 workgroups run in one
// round instead of two.
//
// Arguments: what the first loads need comes first and is preloaded into
// scalar registers at wave launch (the first 14 argument words, built with
// -amdgpu-kernarg-preload-count): weights, scales, exponent bounds, the input
// (x, or the accumulator) and its second operand (gamma, or the SiLU norm
// partials), K, the tile count, the item count with the XCD-order flag in
// bit 31, and ss_n | norm_n << 8. The rest is read from the GemvParams block,
// whose loads go out behind the input loads and are first waited for after
// the weights have been issued (no kernarg_warm here: its wait would come
// first). The item mapping is branch-free, which keeps the compiler from
// hoisting the block's loads, and a wait for them, above the first loads.
template <int GW, int KW, int PRO>
__global__ __launch_bounds__(256) void gemv_q4m4_kernel(const uint8_t* tw, const uint16_t* ts, const int8_t* tes,
                                                        const void* xin, const void* xaux, uint32_t k, uint32_t tiles_a,
                                                        uint32_t items_x, uint32_t ss_nn, GemvParams p) {
    constexpr int NW = 4;
    constexpr int NKB = KW / 64, NZ = GW * KW / 64;
    constexpr int RW = KW / NW;              // input rows per wave (16..128)
    constexpr int RPL = (RW + kWave - 1) / kWave;
    static_assert(KW % 64 == 0 && KW <= 512, "slice of 64..512 rows");
    static_assert(PRO == PRO_PLAIN || PRO == PRO_GAMMA_FIXED || PRO == PRO_SILU_FIXED, "no attention merge here");
    const long long* xacc = static_cast<const long long*>(xin);
    const uint32_t ss_n = ss_nn & 0xFFu, norm_n = ss_nn >> 8;
    __shared__ __align__(16) float xs[KW];
    __shared__ float wred[2][NW];
    __shared__ __align__(16) uint8_t zl[NW][GW][4][KW];
    __shared__ __align__(16) uint8_t zero16[16];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    uint32_t tiles = __builtin_amdgcn_readfirstlane(tiles_a);
    sgpr_pin(tiles);
    const uint32_t item = blockIdx.x + (items_x >> 31) * (xcd_item(blockIdx.x, items_x & 0x7FFFFFFFu) - blockIdx.x);
    const uint32_t tile = item % tiles, split = item / tiles;
    const uint32_t k0 = split * (uint32_t)KW;
    const uint32_t k1 = min(k, k0 + (uint32_t)KW);

    // (the accumulator this launch clears is cleared at the end: on gfx9 a
    // store counts in vmcnt like a load, so stores issued first would hold
    // up every wait for the input rows and weights)

    // ---- this wave's input rows [wave * RW, wave * RW + RW) of the slice ----
    float xp[RPL], ssp = 0.f;
    long long xa[RPL], xb[RPL];
    uint16_t gm[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        const uint32_t row = (uint32_t)(wave * RW + lane + kWave * r);
        const uint32_t rc = min(k0 + row, k - 1u);
        if constexpr (PRO == PRO_PLAIN) xp[r] = static_cast<const float*>(xin)[rc];
        if constexpr (PRO == PRO_GAMMA_FIXED) {
            xa[r] = xacc[rc];
            gm[r] = static_cast<const uint16_t*>(xaux)[rc];
        }
        if constexpr (PRO == PRO_SILU_FIXED) {
            xa[r] = xacc[rc];
            xb[r] = xacc[k + rc];
        }
    }
    if constexpr (PRO == PRO_SILU_FIXED) ssp = static_cast<const float*>(xaux)[min((uint32_t)lane, ss_n - 1u)];
    __builtin_amdgcn_sched_barrier(0);   // the input loads are issued before the weight stream

    // ---- then the wave's scales and weights ----
    uint4 wq[GW][NKB];
    uint32_t sw[(NZ + 1) / 2];
    int esg[GW];
    gemv_q4m_load_scales<GW, NZ>(ts, tes, (uint64_t)item * NW + wave, lane, sw, esg);
    gemv_q4m_load_weights<GW, NKB>(tw, (uint64_t)item * NW + wave, lane, wq);
    __builtin_amdgcn_sched_barrier(0);
    const GemvOut<GW> out = gemv_q4m_out<GW>(p, tile, wave);
    float* ss_dst = nullptr;
    if constexpr (PRO == PRO_GAMMA_FIXED) ss_dst = sgpr_ptr(p.ss_out);

    // ---- x of the wave's rows into LDS, max |x|, sum x^2 ----
    float inv = 1.f;
    if constexpr (PRO == PRO_SILU_FIXED)
        inv = 1.0f / sqrtf(wave_sum(lane < (int)ss_n ? ssp : 0.f) / (float)norm_n + 1e-6f);
    float mx = 0.f, ss = 0.f;
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        const uint32_t lr = (uint32_t)(lane + kWave * r);
        const uint32_t row = (uint32_t)(wave * RW) + lr;
        const bool ok = lr < (uint32_t)RW && k0 + row < k1;
        float x;
        if constexpr (PRO == PRO_PLAIN) {
            x = ok ? xp[r] : 0.f;
        } else if constexpr (PRO == PRO_GAMMA_FIXED) {
            const float xf = ok ? from_fixed(xa[r]) : 0.f;
            fix_flag(out.flag, ok && fix_out_of_range(xa[r], kFixReadLimit));
            ss += xf * xf;
            x = xf * h2f(gm[r]);
        } else {
            x = ok ? silu_mul(inv * from_fixed(xa[r]), inv * from_fixed(xb[r])) : 0.f;
        }
        if (lr < (uint32_t)RW) xs[row] = x;
        mx = fmaxf(mx, fabsf(x));
    }
    mx = wave_max(mx);
    if constexpr (PRO == PRO_GAMMA_FIXED) ss = wave_sum(ss);
    if (lane == 0) {
        wred[0][wave] = mx;
        wred[1][wave] = ss;
    }
    if (wave == 0 && lane < 4) reinterpret_cast<uint32_t*>(zero16)[lane] = 0u;
    __syncthreads();
    const float xm = fmaxf(fmaxf(wred[0][0], wred[0][1]), fmaxf(wred[0][2], wred[0][3]));
    if constexpr (PRO == PRO_GAMMA_FIXED) {
        // the slice's sum of squares (the waves' partials in order), for the
        // consumer of this GEMV's output, which applies the RMSNorm factor
        if (t == 0 && tile == 0)
            __hip_atomic_store(ss_dst + split, ((wred[1][0] + wred[1][1]) + wred[1][2]) + wred[1][3], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    gemv_q4m_item<GW, KW>(out, lane, [](int, uint32_t r) { return xs[r]; }, xm, sw, esg, wq, zl[wave], zero16);
    if (p.zero_ptr)
        for (uint32_t i = blockIdx.x * (NW * kWave) + t; i < p.zero_n; i += gridDim.x * (NW * kWave)) p.zero_ptr[i] = 0;
}

}  // namespace qora
