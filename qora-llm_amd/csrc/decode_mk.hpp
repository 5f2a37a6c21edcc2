// One decode step as a single persistent launch (decode_mk_kernel).
//
// The graph path runs 5 kernels per layer; each launch pays its ramp, its
// first-load latency and its drain, and no kernel can fetch its weights
// before the previous one has finished. Here every workgroup stays resident
// for the whole step and walks the same phase sequence
//   embed, 36 x (q|k|v, attention, o, gate|up, down), lm_head
// issuing each phase's weight loads before it waits for that phase's
// inputs, so the weight stream overlaps the dependency wait.
//
// Synchronisation is carried by the data. Every accumulator element is an
// int64 (value * 2^28) * 256 + count: each producer adds its contribution
// with count 1 in one atomic, and a consumer polls the elements it needs
// until their low byte equals the number of producers. No barrier, no
// counter shared by the whole grid. Cross-workgroup data is only written by
// device-scope atomics (or atomic stores) and read by device-scope atomic
// loads, which the memory model keeps coherent across the XCDs without
// cache-wide write-back or invalidation; a producer waits for its own
// stores (s_waitcnt) before it signals. Every wait is bounded: on a
// timeout the workgroup sets *err and every later wait returns at once, so
// all waves exit and the host reports the error.
//
// Buffers come in two parities (position & 1): a step uses one and clears
// the other for the next step.
//
// Workgroup: 4 matrix-core waves + 1 control wave (320 threads). The control
// wave polls inputs and builds each GEMV slice's input vector in LDS; it
// issues no weight loads, so its polls never queue behind the weight
// stream (a wave's loads complete in issue order).
#pragma once

#include "attn.hpp"
#include "common.hpp"
#include "gemv.hpp"
#include "gemv_mfma.hpp"
#include "lmhead_mfma.hpp"
#include "params.hpp"

namespace qora {

constexpr int kMkNW = 4;                   // matrix-core waves
constexpr int kMkNT = (kMkNW + 1) * 64;    // + control wave
constexpr double kMkScale = 268435456.0;   // 2^28
constexpr double kMkSsScale = 1048576.0;   // 2^20: sums of squares (up to ~3e10 per slice)
constexpr uint32_t kMkSpin = 1u << 22;     // polls before a wait gives up

// ---- counted fixed point ----
__device__ __forceinline__ long long mk_ld(const long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t mk_ld32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float mk_ldf(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void mk_stf(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float mk_value(long long a) {
    return (float)((double)(a >> 8) * (1.0 / kMkScale));
}
__device__ __forceinline__ long long mk_units(double v) {
    return __double2ll_rn(v * kMkScale);
}
// add `units` (value * 2^28) with count 1
__device__ __forceinline__ void mk_add(long long* p, long long units) {
    atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)(units * 256 + 1));
}
// Optional timeline (MkParams::trace): stamp k of phase ph of this workgroup.
__device__ __forceinline__ void mk_stamp(const MkParams& p, uint32_t ph, int k) {
    if (p.trace && threadIdx.x == 0)
        p.trace[((uint64_t)blockIdx.x * (p.nl * 5 + 2) + ph) * 3 + k] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ bool mk_failed(const uint32_t* err) {
    return mk_ld32(err) != 0u;
}
__device__ __forceinline__ void mk_fail(uint32_t* err) {
    __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wait that timed out: err[0] = 1; err[1] counts the reports and entry
// i < 15 at err[2 + 4 i] = wait site (layer << 8 | site code), workgroup,
// element, count seen | count wanted << 16.
__device__ __forceinline__ void mk_report(uint32_t* err, uint32_t site, uint32_t elem, uint32_t got, uint32_t want) {
    __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t i = __hip_atomic_fetch_add(err + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (i == 0u) __hip_atomic_store(err + 201, mk_ld32(err + 200), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (i < 15u) {
        const uint32_t d[4] = {site, blockIdx.x, elem, got | (want << 16)};
#pragma unroll
        for (int k = 0; k < 4; ++k) __hip_atomic_store(err + 2 + 4 * i + k, d[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Wave-level wait until elements [0, n) of src (lane l: l + 64 j) all carry
// count `want`; returns their values (count bits included). False on error.
template <int PL>
__device__ __forceinline__ bool mk_poll(const long long* src, uint32_t n, uint32_t want, long long (&v)[PL],
                                        uint32_t* err, uint32_t site) {
    const uint32_t lane = threadIdx.x & 63u;
    for (uint32_t spins = 0;; ++spins) {
        int ok = 1;
#pragma unroll
        for (int j = 0; j < PL; ++j) {
            const uint32_t i = lane + 64u * (uint32_t)j;
            v[j] = i < n ? mk_ld(src + i) : 0;
            ok &= (i >= n) || ((uint32_t)(v[j] & 0xFF) == want);
        }
        const unsigned long long bad = __ballot(!ok);
        if (bad == 0ull) return true;
        if (spins > kMkSpin || mk_failed(err)) {
            if (spins > kMkSpin && lane == (uint32_t)__builtin_ctzll(bad)) {
                uint32_t elem = 0, got = 0;
#pragma unroll
                for (int j = PL - 1; j >= 0; --j) {
                    const uint32_t i = lane + 64u * (uint32_t)j;
                    if (i < n && (uint32_t)(v[j] & 0xFF) != want) {
                        elem = i;
                        got = (uint32_t)(v[j] & 0xFF);
                    }
                }
                mk_report(err, site, elem, got, want);
            }
            mk_fail(err);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Wave-level wait until a counter reaches `want`.
__device__ __forceinline__ bool mk_wait_u32(const uint32_t* c, uint32_t want, uint32_t* err, uint32_t site) {
    for (uint32_t spins = 0;; ++spins) {
        const uint32_t v = mk_ld32(c);
        if (v >= want) return true;
        if (spins > kMkSpin || mk_failed(err)) {
            if (spins > kMkSpin && (threadIdx.x & 63u) == 0u) mk_report(err, site, 0u, v, want);
            mk_fail(err);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// ---- shared memory of the persistent workgroup ----
struct MkSmem {
    // GEMV phases
    float xs[kMkSlots][kMkKW];
    uint8_t zl[kMkNW][kMkSlots][4][kMkKW];
    uint8_t zero16[16];
    int ex[kMkSlots];          // block exponent of input slice i
    int xsi[kMkSlots];         // item slot -> its input slice
    int abort_;
    int last_;
    // attention
    float ktile[kAttnSub * (128 + 4)];
    float vtile[kAttnSub * 128];
    float qs[kAttnMaxGroups * 128];
    float es[kAttnMaxGroups * kAttnSub];
    float kapp[128], vapp[128];
    float aw[kAttnMaxGroups * kAttnMaxSplits];
    // lm_head
    uint8_t xl[32 * 272];
    float red[8];
    float s_val[kMkNW];
    uint32_t s_idx[kMkNW];
};

// ---- GEMV phase: weights of the workgroup's items ----
struct MkW {
    uint4 wq[kMkSlots][kMkKW / 64];
    uint32_t sw[kMkSlots][(kMkKW / 64 + 1) / 2];
    int es[kMkSlots];
};

__device__ __forceinline__ uint32_t mk_items(const GemvParams& g) {
    return g.tiles * g.splits;
}

// This workgroup's items of a phase: a balanced contiguous range of the
// split-major order (item b: tile b % tiles, K slice b / tiles), so its items
// share one or two K slices.
struct MkRange {
    uint32_t start, count;
};
__device__ __forceinline__ MkRange mk_range(uint32_t items) {
    const uint32_t s = (uint32_t)(((uint64_t)blockIdx.x * items) / gridDim.x);
    const uint32_t e = (uint32_t)(((uint64_t)(blockIdx.x + 1) * items) / gridDim.x);
    return MkRange{s, e - s};
}

// matrix-core wave `wave`: issue the loads of its part of every item
__device__ __forceinline__ void mk_gemv_load(const GemvParams& g, const uint8_t* tw, const uint16_t* ts,
                                             const int8_t* te, int wave, int lane, MkW& w, MkRange rg) {
    constexpr int NKB = kMkKW / 64, NZ = kMkKW / 64;
#pragma unroll
    for (int j = 0; j < kMkSlots; ++j) {
        if ((uint32_t)j >= rg.count) break;
        const uint32_t b = rg.start + (uint32_t)j;
        const uint64_t bw = (uint64_t)b * kMkNW + (uint32_t)wave;
        const uint16_t* sp = ts + (bw * 64u + (uint32_t)lane) * NZ;
        const uint2 sv = *reinterpret_cast<const uint2*>(sp);
        w.sw[j][0] = sv.x;
        w.sw[j][1] = sv.y;
        w.es[j] = __builtin_amdgcn_readfirstlane((int)te[bw]);
        const uint8_t* wp = tw + bw * (uint64_t)(NKB * 1024) + (uint32_t)lane * 16u;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) w.wq[j][kb] = *reinterpret_cast<const uint4*>(wp + kb * 1024);
    }
}

// matrix-core wave, item slot j: z = x * s quantised to 30-bit limbs in LDS
__device__ __forceinline__ void mk_gemv_quant(int wave, int lane, const MkW& w, int j, MkSmem& sm) {
    constexpr int NZ = kMkKW / 64;
    const int xi = sm.xsi[j];
    const int ex = sm.ex[xi];
    const int es = w.es[j];
    const float* xs = sm.xs[xi];
    uint8_t* zl = &sm.zl[wave][j][0][0];
#pragma unroll
    for (int u = 0; u < NZ; ++u) {
        const uint32_t rz = (uint32_t)lane * NZ + u;
        const uint16_t sbits = (uint16_t)((u & 1) ? (w.sw[j][u / 2] >> 16) : (w.sw[j][u / 2] & 0xFFFFu));
        const float z = xs[rz] * h2f(sbits);
        const int M = (int)rintf(ldexpf(z, 30 - (ex + es)));
        const uint32_t limbs = (uint32_t)(M + 0x808080) ^ 0x808080u;
        zl[rz] = (uint8_t)(limbs & 0xFFu);
        zl[kMkKW + rz] = (uint8_t)((limbs >> 8) & 0xFFu);
        zl[2 * kMkKW + rz] = (uint8_t)((limbs >> 16) & 0xFFu);
        zl[3 * kMkKW + rz] = (uint8_t)(limbs >> 24);
    }
}

// matrix-core wave, item slot j: C[limb][column] = A[limb][k] * B[k][column]
__device__ __forceinline__ void mk_gemv_mfma(int wave, int lane, const MkW& w, int j, const MkSmem& sm, v4i32 (&acc)[2]) {
    constexpr int NKB = kMkKW / 64;
    const uint8_t* zl = &sm.zl[wave][j][0][0];
    acc[0] = (v4i32){0, 0, 0, 0};
    acc[1] = (v4i32){0, 0, 0, 0};
    const uint32_t li = (uint32_t)lane % 16, lk = (uint32_t)lane / 16;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        const uint8_t* ap = li < 4 ? zl + li * kMkKW + kb * 64 + 16 * lk : sm.zero16;
        const v4i32 a = *reinterpret_cast<const v4i32*>(ap);
        const uint4 wv = w.wq[j][kb];
        acc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, q4_bfrag(wv.x, wv.y), acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, q4_bfrag(wv.z, wv.w), acc[1], 0, 0, 0);
    }
}

// matrix-core wave, item b in slot j: value = Y * 2^(E - 34); in 2^28 units
// Y << (E - 6), rounded when negative; added with count 1 per column
__device__ __forceinline__ void mk_gemv_epilogue(const GemvParams& g, uint32_t b, int wave, int lane, const MkW& w,
                                                 int j, const MkSmem& sm, const v4i32 (&acc)[2], long long* out) {
    if (lane >= 16) return;
    const uint32_t tile = b % g.tiles;
    const LaneSrc src = lane_source(g, tile, wave, 4);
    if (src.grp >= src.sg.groups) return;
    const int sh = max(min(sm.ex[sm.xsi[j]] + w.es[j] - 6, 62), -62);
    const int rsh = sh < 0 ? -sh : 0, lsh = sh > 0 ? sh : 0;
    const long long rnd = rsh > 0 ? (1LL << (rsh - 1)) : 0;
    long long* dst = out + src.sg.col0 + src.grp * 32u + (uint32_t)lane;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const v4i32 c = acc[h];
        const int lo = c[0] + (c[1] << 8);
        const int hi = c[2] + (c[3] << 8);
        const long long Y = (long long)lo + ((long long)hi << 16);
        mk_add(dst + h * 16, ((Y + rnd) >> rsh) << lsh);
    }
}

// control wave: block exponent of a slice from max |x| (0 for all zeros)
__device__ __forceinline__ int mk_exponent(float mx) {
    return mx > 0.f ? (int)((__float_as_uint(mx) >> 23) & 0xFFu) - 126 : 0;
}


// ---------------------------------------------------------------------------
// GEMV phases. Item b (= the standalone kernel's block index: tile b % tiles,
// K slice b / tiles) belongs to workgroup b % gridDim.x, slot b / gridDim.x.
// ---------------------------------------------------------------------------

// control wave: input slice of item b into sm.xs[j] and sm.ex[j]
//   MK_QKV / MK_GU: x * gamma of the counted residual rows (RMSNorm factor
//     applied by the consumer); column-tile-0 items add sum(x^2) to *ss_out
//   MK_DOWN: silu(inv g) * (inv u) of the counted gate|up rows
//   MK_O: rows of the merged attention output, once its heads are flagged
// Returns false on a failed wait.
template <int KIND>
__device__ __forceinline__ bool mk_gemv_input(const MkParams& p, const GemvParams& g, uint32_t b, int j,
                                              const long long* in, uint32_t want, const uint16_t* gamma,
                                              long long* ss_out, const long long* ss_in, uint32_t ss_want,
                                              const uint32_t* flags, MkSmem& sm, uint32_t site) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t tile = b % g.tiles, split = b / g.tiles;
    const uint32_t k0 = split * kMkKW;
    const uint32_t n = min((uint32_t)kMkKW, g.k - k0);
    float* xs = sm.xs[j];
    float mx = 0.f;
    if constexpr (KIND == MK_QKV || KIND == MK_GU) {
        long long v[4];
        if (!mk_poll<4>(in + k0, n, want, v, p.err, site | (KIND * 16 + 1))) return false;
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t i = lane + 64u * q;
            float x = 0.f;
            if (i < n) {
                const float xf = mk_value(v[q]);
                ss += xf * xf;
                x = xf * h2f(gamma[k0 + i]);
            }
            xs[i] = x;
            mx = fmaxf(mx, fabsf(x));
        }
        ss = wave_sum(ss);
        if (tile == 0 && lane == 0) mk_add(ss_out, __double2ll_rn((double)ss * kMkSsScale));

    } else if constexpr (KIND == MK_DOWN) {
        long long gv[4], uv[4], sv[1];
        if (!mk_poll<1>(ss_in, 1, ss_want, sv, p.err, site | (KIND * 16 + 2))) return false;
        if (!mk_poll<4>(in + k0, n, want, gv, p.err, site | (KIND * 16 + 3))) return false;
        if (!mk_poll<4>(in + p.inter + k0, n, want, uv, p.err, site | (KIND * 16 + 4))) return false;
        const float ssum = (float)((double)(__shfl(sv[0], 0, 64) >> 8) * (1.0 / kMkSsScale));
        const float inv = 1.0f / sqrtf(ssum / (float)p.hidden + 1e-6f);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t i = lane + 64u * q;
            const float x = i < n ? silu_mul(inv * mk_value(gv[q]), inv * mk_value(uv[q])) : 0.f;
            xs[i] = x;
            mx = fmaxf(mx, fabsf(x));
        }
    } else {
        // attention output rows [k0, k0 + n): merge of the split partials of the
        // heads they belong to (online-softmax merge in split order, as
        // attn_merge_rows_wave), once every split of their KV heads is counted
        const uint32_t hd = p.hd, G = p.G;
        const uint32_t L = (uint32_t)(*p.pos) + 1u;
        const uint32_t s_act = min(p.s_max, (L + p.chunk - 1) / p.chunk);
        const uint32_t h0 = k0 / hd, h1 = (k0 + n - 1) / hd;
        for (uint32_t kv = h0 / G; kv <= h1 / G; ++kv)
            if (!mk_wait_u32(flags + kv, s_act, p.err, site | (KIND * 16 + 5))) return false;
        const uint64_t sstride = (uint64_t)G * (hd + 2);
        // per-head split weights: lane s holds split s
        const uint32_t nh = h1 - h0 + 1;   // <= 4
        const uint32_t sc = min(lane, s_act - 1u);
        const bool sok = lane < s_act;
        for (uint32_t hh = 0; hh < nh; ++hh) {
            const uint32_t h = h0 + hh;
            const float* base = p.part + ((uint64_t)(h / G) * p.s_max + sc) * sstride + (uint64_t)(h % G) * (hd + 2);
            const float ms = mk_ldf(base + hd), ls = mk_ldf(base + hd + 1);
            const float mm = wave_max(sok ? ms : -INFINITY);
            const float wgt = sok ? expf(ms - mm) : 0.f;
            const float den = wave_sum(sok ? ls * wgt : 0.f);
            sm.aw[hh * kAttnMaxSplits + lane] = sok ? wgt / den : 0.f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t i = lane + 64u * q;
            float x = 0.f;
            if (i < n) {
                const uint32_t r = k0 + i, h = r / hd, d = r % hd, hh = h - h0;
                const float* base = p.part + (uint64_t)(h / G) * p.s_max * sstride + (uint64_t)(h % G) * (hd + 2) + d;
                float pv[8];
                for (uint32_t s0 = 0; s0 < s_act; s0 += 8) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) pv[u] = mk_ldf(base + (uint64_t)min(s0 + u, s_act - 1u) * sstride);
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        x = s0 + u < s_act ? fmaf(pv[u], sm.aw[hh * kAttnMaxSplits + s0 + u], x) : x;
                }
            }
            xs[i] = x;
            mx = fmaxf(mx, fabsf(x));
        }
    }
    mx = wave_max(mx);
    if (lane == 0) sm.ex[j] = mk_exponent(mx);
    return true;
}

// control wave: residual carry of a K-slice-0 item: out[col] += prev[col] for
// the item's columns (the prev vector is complete: count prev_want)
__device__ __forceinline__ bool mk_carry(const MkParams& p, const GemvParams& g, uint32_t b, const long long* prev,
                                         uint32_t prev_want, long long* out, uint32_t site) {
    const uint32_t tile = b % g.tiles;
    if (b / g.tiles != 0) return true;
    const uint32_t c0 = tile * 128u;
    const uint32_t n = min(128u, p.hidden - c0);
    long long v[2];
    if (!mk_poll<2>(prev + c0, n, prev_want, v, p.err, site)) return false;
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t i = lane + 64u * q;
        if (i < n) mk_add(out + c0 + i, v[q] >> 8);
    }
    return true;
}

// One GEMV phase. Returns false if the workgroup must stop (a failed wait).
template <int KIND>
__device__ __forceinline__ bool mk_gemv_phase(const MkParams& p, const MkLayer& ly, const long long* in, uint32_t want,
                                              long long* out, const long long* ss_in, uint32_t ss_want,
                                              long long* ss_out, const uint32_t* flags,
                                              const long long* carry_prev, uint32_t carry_want, MkSmem& sm,
                                              uint32_t l) {
    const GemvParams& g = p.g[KIND];
    const uint32_t site = l << 8;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const MkRange rg = mk_range(mk_items(g));
    MkW w;
    const uint32_t ph = 1 + l * 5 + (KIND == MK_QKV ? 0 : KIND + 1);
    mk_stamp(p, ph, 0);
    if (wave < kMkNW) {
        mk_gemv_load(g, ly.tw[KIND], ly.ts[KIND], ly.te[KIND], wave, lane, w, rg);
    } else {
        // one input slice per distinct K slice of the range (the first item of
        // a slice in split-major order is the only one that can be its tile 0)
        bool ok = true;
        int nx = 0;
        uint32_t prev_split = 0xFFFFFFFFu;
        for (uint32_t j = 0; j < rg.count && ok; ++j) {
            const uint32_t b = rg.start + j;
            const uint32_t split = b / g.tiles;
            if (split != prev_split) {
                const uint16_t* gm = KIND == MK_QKV ? ly.gamma[0] : ly.gamma[1];
                ok = mk_gemv_input<KIND>(p, g, b, nx, in, want, gm, ss_out, ss_in, ss_want, flags, sm, site);
                prev_split = split;
                ++nx;
            }
            if (lane == 0) sm.xsi[j] = nx - 1;
            if (ok && (KIND == MK_O || KIND == MK_DOWN))
                ok = mk_carry(p, g, b, carry_prev, carry_want, out, site | (KIND * 16 + 6));
        }
        if (lane == 0) sm.abort_ = ok ? 0 : 1;
    }
    __syncthreads();
    mk_stamp(p, ph, 1);
    if (sm.abort_) return false;
    if (wave < kMkNW) {
        // all items' quantisation, then all their MFMA chains, then the epilogues
#pragma unroll
        for (int j = 0; j < kMkSlots; ++j)
            if ((uint32_t)j < rg.count) mk_gemv_quant(wave, lane, w, j, sm);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        v4i32 acc[kMkSlots][2];
#pragma unroll
        for (int j = 0; j < kMkSlots; ++j)
            if ((uint32_t)j < rg.count) mk_gemv_mfma(wave, lane, w, j, sm, acc[j]);
#pragma unroll
        for (int j = 0; j < kMkSlots; ++j)
            if ((uint32_t)j < rg.count) mk_gemv_epilogue(g, rg.start + (uint32_t)j, wave, lane, w, j, sm, acc[j], out);
    }
    __syncthreads();   // xs / zl are rewritten by the next phase
    mk_stamp(p, ph, 2);
    return true;
}

// ---------------------------------------------------------------------------
// Attention phase: item (kvh, split) = workgroup kvh * s_act + split.
// Writes its partial, counts itself in A[kvh]; the last item of a KV head
// merges the partials (in split order) into AO and sets F[kvh].
// ---------------------------------------------------------------------------
template <int DPL, bool F16KV>
__device__ __forceinline__ bool mk_attn_phase(const MkParams& p, const MkLayer& ly, uint32_t l, const MkBufs& bf,
                                              uint32_t L, uint32_t s_act, uint32_t qkv_want, MkSmem& sm) {
    constexpr int NTT = 256;                         // threads that load tiles (waves 0..3)
    constexpr int SUB = kAttnSub;
    constexpr int HDM = 64 * DPL;
    constexpr int KQ = HDM / 8;
    constexpr int KSTR = HDM + 4;
    constexpr int VSTR = HDM;
    constexpr int TL = SUB * HDM / 4 / NTT;
    const uint32_t item = blockIdx.x;
    if (item >= p.KVH * s_act) return true;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t / 64;
    const uint32_t kvh = item / s_act, split = item % s_act;
    const uint32_t hd = p.hd, G = p.G, nq = G * hd, qd = p.H * hd;
    const uint64_t kv_stride = (uint64_t)p.KVH * hd;    // q|k|v accumulator layout
    const uint64_t head_off = (uint64_t)kvh * hd;
    const uint64_t cps = p.kv_ps, coff = (uint64_t)kvh * p.kv_hs;   // cache layout
    const uint32_t p0 = split * p.chunk;
    const uint32_t p1 = min(L, p0 + p.chunk);
    const uint32_t cur = L - 1;
    const bool has_new = cur >= p0 && cur < p1;
    const uint32_t q4_row = hd / 4, tile_n = SUB * q4_row;
    AttnParams ap{};
    ap.kc = ly.kc;
    ap.vc = ly.vc;
    ap.KVH = p.KVH;
    ap.hd = hd;
    // waves 0..3: the first cache tile (independent of this step's q, k, v)
    KvTileRegs<TL> tr;
    if (t < NTT) tr = attn_load_tile<TL, F16KV>(ap, threadIdx.x, p0, L, cps, coff, q4_row, tile_n);
    const long long* Qb = bf.Q + (uint64_t)l * (qd + 2 * kv_stride);
    if (wave == kMkNW) {
        // control wave: q of the group's heads and the appended k, v, normalised and rotated
        // one wait over every input: RMSNorm sum, q of the group, k, v
        bool ok = true;
        long long sv[1], qv[8], kv2[2], vv2[2];
        for (uint32_t spins = 0;; ++spins) {
            int good = 1;
            sv[0] = lane == 0 ? mk_ld(bf.SS + 2 * l) : 0;
            good &= lane != 0 || (uint32_t)(sv[0] & 0xFF) == qkv_want;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t i = (uint32_t)lane + 64u * q;
                qv[q] = i < nq ? mk_ld(Qb + (uint64_t)kvh * nq + i) : 0;
                good &= i >= nq || (uint32_t)(qv[q] & 0xFF) == qkv_want;
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t i = (uint32_t)lane + 64u * q;
                kv2[q] = i < hd ? mk_ld(Qb + qd + head_off + i) : 0;
                vv2[q] = i < hd ? mk_ld(Qb + qd + kv_stride + head_off + i) : 0;
                good &= i >= hd || ((uint32_t)(kv2[q] & 0xFF) == qkv_want && (uint32_t)(vv2[q] & 0xFF) == qkv_want);
            }
            const unsigned long long bad = __ballot(!good);
            if (bad == 0ull) break;
            if (spins > kMkSpin || mk_failed(p.err)) {
                if (spins > kMkSpin && lane == (int)__builtin_ctzll(bad)) mk_report(p.err, (l << 8) | 0x42, kvh, 0, qkv_want);
                mk_fail(p.err);
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (ok) {
            const float ssum = (float)((double)(__shfl(sv[0], 0, 64) >> 8) * (1.0 / kMkSsScale));
            const float inv = 1.0f / sqrtf(ssum / (float)p.hidden + 1e-6f);
            for (uint32_t i = (uint32_t)lane; i < G * HDM; i += 64) sm.qs[i] = 0.f;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t i = (uint32_t)lane + 64u * q;
                if (i < nq) sm.qs[(i / hd) * HDM + i % hd] = inv * mk_value(qv[q]);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t i = (uint32_t)lane + 64u * q;
                if (i < hd) {
                    sm.kapp[i] = inv * mk_value(kv2[q]);
                    sm.vapp[i] = inv * mk_value(vv2[q]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (ly.use_rope) {
                // rotate_half pairs (d, d + half) at position cur (apply_rope_raw, gemv.rs:757-778)
                const float* ct = p.rope_cos + (uint64_t)cur * p.half;
                const float* st = p.rope_sin + (uint64_t)cur * p.half;
                for (uint32_t e = (uint32_t)lane; e < (G + 1) * p.half; e += 64) {
                    const uint32_t hh = e / p.half, d = e % p.half;
                    float* row = hh < G ? sm.qs + hh * HDM : sm.kapp;
                    const float c = ct[d], s = st[d];
                    const float x1 = row[d], x2 = row[d + p.half];
                    row[d] = x1 * c - x2 * s;
                    row[d + p.half] = x2 * c + x1 * s;
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            if (has_new) {
                // the appended row goes into the cache (read by later steps)
                for (uint32_t d = (uint32_t)lane; d < hd; d += 64) {
                    const uint64_t idx = (uint64_t)cur * cps + coff + d;
                    if constexpr (F16KV) {
                        const uint16_t kh = f2h(sm.kapp[d]), vh = f2h(sm.vapp[d]);
                        reinterpret_cast<uint16_t*>(ly.kc)[idx] = kh;
                        reinterpret_cast<uint16_t*>(ly.vc)[idx] = vh;
                        sm.kapp[d] = h2f(kh);
                        sm.vapp[d] = h2f(vh);
                    } else {
                        reinterpret_cast<float*>(ly.kc)[idx] = sm.kapp[d];
                        reinterpret_cast<float*>(ly.vc)[idx] = sm.vapp[d];
                    }
                }
            }
        }
        if (lane == 0) sm.abort_ = ok ? 0 : 1;
    }
    // K padding columns stay zero
    if (hd < (uint32_t)HDM && t < NTT)
        for (uint32_t e = t; e < SUB * ((uint32_t)HDM - hd); e += NTT)
            sm.ktile[(e / ((uint32_t)HDM - hd)) * KSTR + hd + e % ((uint32_t)HDM - hd)] = 0.f;
    __syncthreads();
    if (sm.abort_) return false;

    const uint32_t g = (uint32_t)wave;
    const uint32_t half_id = (uint32_t)lane / 32, r_lane = (uint32_t)lane % 32;
    const uint32_t dq0 = half_id * (HDM / 2);
    const uint32_t dv0c = min((uint32_t)lane * DPL, hd - DPL);
    const bool vlane = (uint32_t)lane * DPL < hd;
    const float scale = 1.0f / sqrtf((float)hd);
    float m = -INFINITY, lsum = 0.f;
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    for (uint32_t c0 = p0; c0 < p1; c0 += SUB) {
        const uint32_t cn = min((uint32_t)SUB, p1 - c0);
        const bool new_here = has_new && cur >= c0 && cur < c0 + cn;
        if (t < NTT) {
            // attn_store_tile indexes by threadIdx.x < 256
            attn_store_tile<TL, KSTR, VSTR>(tr, threadIdx.x, sm.ktile, sm.vtile, cn, new_here ? cur - c0 : 0xFFFFFFFFu, q4_row,
                                            tile_n);
            if (new_here && (uint32_t)t < hd) {
                sm.ktile[(cur - c0) * KSTR + t] = sm.kapp[t];
                sm.vtile[(cur - c0) * VSTR + t] = sm.vapp[t];
            }
        }
        __syncthreads();
        if (c0 + SUB < p1 && t < NTT)
            tr = attn_load_tile<TL, F16KV>(ap, threadIdx.x, c0 + SUB, L, cps, coff, q4_row, tile_n);
        if (g < G) {
            const float* qg = sm.qs + g * HDM + dq0;
            const float* krow = sm.ktile + r_lane * KSTR + dq0;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            // four float4 pairs at a time: the whole row in registers would cost 128 VGPRs
#pragma unroll
            for (int i0 = 0; i0 < KQ; i0 += 4) {
                float4 q4[4], k4[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    q4[i] = *reinterpret_cast<const float4*>(qg + 4 * (i0 + i));
                    k4[i] = *reinterpret_cast<const float4*>(krow + 4 * (i0 + i));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a0 = fmaf(q4[i].x, k4[i].x, a0);
                    a1 = fmaf(q4[i].y, k4[i].y, a1);
                    a2 = fmaf(q4[i].z, k4[i].z, a2);
                    a3 = fmaf(q4[i].w, k4[i].w, a3);
                }
            }
            float sc = (a0 + a1) + (a2 + a3);
            sc += __shfl_xor(sc, 32, kWave);
            sc = (r_lane < cn) ? sc * scale : -INFINITY;
            const float m_new = fmaxf(m, wave_max(sc));
            const float f = expf(m - m_new);
            const float e = (r_lane < cn) ? expf(sc - m_new) : 0.f;
            lsum = lsum * f + wave_sum(half_id == 0 ? e : 0.f);
            m = m_new;
            if (half_id == 0) sm.es[g * SUB + r_lane] = e;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[i] *= f;
#pragma unroll 8
            for (int r = 0; r < SUB; ++r) {
                const float er = sm.es[g * SUB + r];
                const float* vrow = sm.vtile + r * VSTR + dv0c;
                if constexpr (DPL == 2) {
                    const float2 v2 = *reinterpret_cast<const float2*>(vrow);
                    acc[0] = fmaf(er, v2.x, acc[0]);
                    acc[1] = fmaf(er, v2.y, acc[1]);
                } else {
                    acc[0] = fmaf(er, vrow[0], acc[0]);
                }
            }
        }
        __syncthreads();
    }
    // partial of (kvh, split, g), then count this item (the o phase merges)
    const uint64_t sstride = (uint64_t)G * (hd + 2);
    if (g < G) {
        float* part = p.part + ((uint64_t)kvh * p.s_max + split) * sstride + (uint64_t)g * (hd + 2);
        if (vlane) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) mk_stf(part + dv0c + i, acc[i]);
        }
        if (lane == 0) {
            mk_stf(part + hd, m);
            mk_stf(part + hd + 1, lsum);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0)
        __hip_atomic_fetch_add(bf.A + (uint64_t)l * p.KVH + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// ---------------------------------------------------------------------------
// lm_head phase (lmhead_q4m_kernel's scheme): the control wave waits for the
// final residual and builds the limb bytes; the matrix-core waves stream
// tiles gw, gw + W, ... (gw = 4 b + wave, W = 4 gridDim.x).
// ---------------------------------------------------------------------------
template <int NP>
__device__ __forceinline__ void mk_lm_phase(const MkParams& p, const long long* R, uint32_t want, MkSmem& sm) {
    constexpr int UPT = NP / 2;
    constexpr int COLS = 64 * NP;
    constexpr int SLOT = 272;
    constexpr int XPL = COLS / 64;               // inputs per lane of the control wave
    const LmHeadParams& lm = p.lm;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const uint32_t W = gridDim.x * kMkNW;
    const uint32_t last = lm.tiles - 1u;
    uint32_t tile = blockIdx.x * kMkNW + (uint32_t)wave;
    uint4 wb[UPT];
    uint32_t sb[UPT];
    if (wave < kMkNW) {
        const uint32_t tl = min(tile, last);
        const uint8_t* wp = lm.tw + (uint64_t)tl * UPT * 1024u + (uint32_t)lane * 16u;
        const uint32_t* sp = lm.ts + (uint64_t)tl * UPT * 32u + ((uint32_t)lane & 31u);
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            wb[u] = *reinterpret_cast<const uint4*>(wp + u * 1024);
            sb[u] = sp[u * 32];
        }
    } else {
        // the final residual, polled 512 values at a time and parked in LDS
        // (the attention tile area is free in this phase)
        float* xp = sm.ktile;
        static_assert(COLS <= kAttnSub * (128 + 4), "lm_head input fits the tile area");
        bool ok = true;
        float ss = 0.f, mx = 0.f;
        for (int c0 = 0; c0 < COLS && ok; c0 += 512) {
            long long v[8];
            ok = mk_poll<8>(R + c0, min(512, COLS - c0), want, v, p.err, 0x50u | ((uint32_t)c0 << 8));
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int c = c0 + lane + 64 * q;
                if (c < COLS) {
                    const float x = mk_value(v[q]);
                    xp[c] = x;
                    ss += x * x;
                }
            }
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)COLS + 1e-6f);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int c = lane; c < COLS; c += 64) {
            const float x = xp[c] * inv * h2f(lm.gamma[c]);
            xp[c] = x;
            mx = fmaxf(mx, fabsf(x));
        }
        mx = wave_max(mx);
        const int ex = mk_exponent(mx);
        for (int q = 0; q < XPL; ++q) {
            const uint32_t c = (uint32_t)(lane + 64 * q);
            const int M = (int)rintf(ldexpf(xp[c], 30 - ex));
            const uint32_t limbs = (uint32_t)(M + 0x808080) ^ 0x808080u;
            uint8_t* dst = sm.xl + (c / 64u) * SLOT + ((c % 64u) / 16u) * 64u + (c % 16u);
            dst[0] = (uint8_t)(limbs & 0xFFu);
            dst[16] = (uint8_t)((limbs >> 8) & 0xFFu);
            dst[32] = (uint8_t)((limbs >> 16) & 0xFFu);
            dst[48] = (uint8_t)(limbs >> 24);
        }
        for (int i = lane; i < NP * 4; i += 64) *reinterpret_cast<uint32_t*>(sm.xl + (i / 4) * SLOT + 256 + (i % 4) * 4) = 0u;
        if (lane == 0) {
            sm.ex[0] = ex;
            sm.abort_ = ok ? 0 : 1;
        }
    }
    __syncthreads();
    if (sm.abort_) return;
    const int ex = sm.ex[0];
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    if (wave < kMkNW) {
        const uint32_t li = (uint32_t)lane % 16u, kq = (uint32_t)lane / 16u;
        const bool nz = li < 8u && (li >> 2) == (kq >> 1);
        const uint32_t aoff = nz ? kq * 64u + (li & 3u) * 16u : 256u;
        const v4i32 zero = (v4i32){0, 0, 0, 0};
        for (; tile < lm.tiles; tile += W) {
            uint32_t ao = aoff;
            asm volatile("" : "+v"(ao));
            const uint32_t nx = min(tile + W, last);
            const uint8_t* wp = lm.tw + (uint64_t)nx * UPT * 1024u + (uint32_t)lane * 16u;
            const uint32_t* sp = lm.ts + (uint64_t)nx * UPT * 32u + ((uint32_t)lane & 31u);
            float acc = 0.f;
#pragma unroll
            for (int u = 0; u < UPT; ++u) {
                const uint4 wv = wb[u];
                const uint32_t s2 = sb[u];
                wb[u] = *reinterpret_cast<const uint4*>(wp + u * 1024);
                sb[u] = sp[u * 32];
                const v4i32 a0 = *reinterpret_cast<const v4i32*>(sm.xl + (2 * u) * SLOT + ao);
                const v4i32 a1 = *reinterpret_cast<const v4i32*>(sm.xl + (2 * u + 1) * SLOT + ao);
                const v4i32 c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, q4_bfrag(wv.x, wv.y), zero, 0, 0, 0);
                const v4i32 c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, q4_bfrag(wv.z, wv.w), zero, 0, 0, 0);
                acc = fmaf(lm_limb_value(c0), f16lo(s2), acc);
                acc = fmaf(lm_limb_value(c1), f16hi(s2), acc);
            }
            acc += __shfl_xor(acc, 16, kWave);
            const float y = ldexpf(acc, ex - 34);
            const uint32_t r = tile * 16u + (uint32_t)lane;
            if (lane < 16 && r < lm.rows) {
                lm.y[r] = y;
                if (argmax_better(y, r, best_v, best_i)) {
                    best_v = y;
                    best_i = r;
                }
            }
        }
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
            sm.s_val[wave] = best_v;
            sm.s_idx[wave] = best_i;
        }
    }
    __syncthreads();
    if (t == 0) {
        float bv = sm.s_val[0];
        uint32_t bi = sm.s_idx[0];
        for (int w2 = 1; w2 < kMkNW; ++w2)
            if (argmax_better(sm.s_val[w2], sm.s_idx[w2], bv, bi)) {
                bv = sm.s_val[w2];
                bi = sm.s_idx[w2];
            }
        lm.part_val[blockIdx.x] = bv;
        lm.part_idx[blockIdx.x] = bi;
    }
}

// ---------------------------------------------------------------------------
// The step. NP: hidden / 64 (lm_head); DPL, F16KV: attention variant.
// ---------------------------------------------------------------------------
// The parameters live in device memory (a by-value kernel argument this large
// is copied to scratch as soon as any member is indexed at run time).
template <int NP, int DPL, bool F16KV>
__global__ __launch_bounds__(kMkNT) void decode_mk_kernel(const MkParams* __restrict__ pp) {
    __shared__ MkSmem sm;
    const MkParams& p = *pp;
    const int t = threadIdx.x;
    const int32_t pos = *p.pos;
    const uint32_t L = (uint32_t)pos + 1u;
    const int par = pos & 1;
    const MkBufs& bf = p.buf[par];
    const uint32_t s_act = min(p.s_max, (L + p.chunk - 1) / p.chunk);

    if (t == 0) __hip_atomic_fetch_add(p.err + 200, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (p.residency_test) {
        if (t == 0) {
            uint32_t v = 0;
            for (uint32_t i = 0; i < (1u << 18); ++i) {
                v = mk_ld32(p.err + 200);
                if (v >= gridDim.x) break;
                __builtin_amdgcn_s_sleep(2);
            }
            // the fewest workgroups any of them saw running: with full residency every
            // one sees the whole grid, otherwise the first ones time out first
            __hip_atomic_fetch_min(p.err + 202, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();   // every wave stays resident while wave 0 waits
        return;
    }
    // clear the other parity for the next step
    {
        uint4* cb = reinterpret_cast<uint4*>(p.clear_base[par ^ 1]);
        for (uint64_t i = (uint64_t)blockIdx.x * kMkNT + t; i < p.clear_n; i += (uint64_t)gridDim.x * kMkNT)
            cb[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (t < 4) reinterpret_cast<uint32_t*>(sm.zero16)[t] = 0u;

    mk_stamp(p, 0, 0);
    // embedding row of this step's token -> R[0] (count 1)
    {
        const uint32_t i = blockIdx.x * kMkNT + t;
        if (i < p.hidden) {
            const int32_t tk = p.with_lm ? *p.token : p.prompt[pos];
            const uint32_t tok = min((uint32_t)max(tk, 0), p.vocab - 1u);
            const uint8_t b = p.emb_w[(uint64_t)tok * (p.hidden / 2) + i / 2];
            const int q = (i & 1) ? (b >> 4) : (b & 0xF);
            const float v = h2f(p.emb_s[(uint64_t)tok * (p.hidden / 32) + i / 32]) * (float)(q - 8);
            mk_add(bf.R + i, mk_units((double)v));
        }
    }

    const uint32_t qkv_n = p.H * p.hd + 2 * p.KVH * p.hd;
    const uint32_t c_qkv = p.g[MK_QKV].splits, c_o = p.g[MK_O].splits + 1;
    const uint32_t c_gu = p.g[MK_GU].splits, c_down = p.g[MK_DOWN].splits + 1;
    for (uint32_t l = 0; l < p.nl; ++l) {
        const MkLayer& ly = p.layers[l];
        const long long* R = bf.R + (uint64_t)l * p.hidden;
        const uint32_t c_r = l == 0 ? 1u : c_down;
        long long* Q = bf.Q + (uint64_t)l * qkv_n;
        long long* RP = bf.RP + (uint64_t)l * p.hidden;
        long long* U = bf.U + (uint64_t)l * 2 * p.inter;
        long long* SS = bf.SS + 2 * l;
        const uint32_t* A = bf.A + (uint64_t)l * p.KVH;   // attention items counted per KV head
        long long* Rn = bf.R + (uint64_t)(l + 1) * p.hidden;
        if (!mk_gemv_phase<MK_QKV>(p, ly, R, c_r, Q, nullptr, 0, SS, nullptr, nullptr, 0, sm, l)) return;
        mk_stamp(p, 1 + l * 5 + 1, 0);
        if (!mk_attn_phase<DPL, F16KV>(p, ly, l, bf, L, s_act, c_qkv, sm)) return;
        __syncthreads();
        mk_stamp(p, 1 + l * 5 + 1, 2);
        if (!mk_gemv_phase<MK_O>(p, ly, nullptr, 0, RP, nullptr, 0, nullptr, A, R, c_r, sm, l)) return;
        if (!mk_gemv_phase<MK_GU>(p, ly, RP, c_o, U, nullptr, 0, SS + 1, nullptr, nullptr, 0, sm, l)) return;
        if (!mk_gemv_phase<MK_DOWN>(p, ly, U, c_gu, Rn, SS + 1, c_gu, nullptr, nullptr, RP, c_o, sm, l)) return;
    }
    if (p.with_lm) {
        mk_stamp(p, 1 + p.nl * 5, 0);
        mk_lm_phase<NP>(p, bf.R + (uint64_t)p.nl * p.hidden, p.nl == 0 ? 1u : c_down, sm);
        mk_stamp(p, 1 + p.nl * 5, 2);
    }
}

}  // namespace qora
