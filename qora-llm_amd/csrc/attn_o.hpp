// Short-context decode: GQA attention and the o projection in one kernel.
//
// The split attention kernel and the o GEMV each pay a launch's fixed
// latency (wave launch, first loads, drain) of a few microseconds, far more
// than their work at a short context. Here the o GEMV's K slice is one query
// head h (KW = head_dim), so a workgroup needs only head h's attention output:
// it computes it itself, from the q|k|v sums of the q|k|v GEMV and the cache,
// and feeds it to the same matrix-core pass as gemv_q4m_kernel (same work
// items, same packed weights). The 16 column tiles of a head repeat its
// attention; at a short context that costs less than a launch.
//
// Chunked (CH, mid contexts): the column tiles of a head split its context
// instead, tile j attending over positions [32 NP j, 32 NP (j + 1)); each
// leaves its chunk's softmax state in global memory, counts it in the head's
// counter, waits (bounded) for the head's other chunks and merges them in
// chunk order before its matrix-core pass (chunk_publish, chunk_merge).
//
// Attention (gemv.rs:914-989, softmax_raw gemv.rs:782-793) of head h over
// KV head h / groups, positions [0, L), L = *pos + 1:
//   * the kernel is compiled per pass count NP (32 positions a pass, contexts
//     32 (NP - 1) < L <= 32 NP; the host picks the variant from the position
//     it appends), so every loop is unrolled to its live passes and only the
//     last pass needs masks. The rows of passes 0 .. NP - 2 lie below the
//     appended position whatever it is: their loads go out before the
//     position arrives;
//   * the arguments of the first loads (cache, position, q|k|v sums, norm
//     partials, shape and strides) come ahead of the parameter block and are
//     preloaded into scalar registers at wave launch: the K rows go out at
//     once, the parameter block's lines with the position, and the RoPE row
//     (whose table pointers are in the block) after the V rows;
//   * q, the appended k row and v row: RMSNorm factor of the q|k|v GEMV input
//     applied to the fixed-point sums, q and k rotated at position L - 1
//     (apply_rope_raw, gemv.rs:903-906); the workgroup of column tile 0 of the
//     group's first head writes the k and v rows into the cache
//     (gemv.rs:909-911), every workgroup uses them from LDS;
//   * all 8 waves take positions: lane (c, j) = (lane % 16, lane / 16) of wave
//     w holds position 32 i + 4 w + j of pass i and dims 64 u + 4 c .. + 3, so
//     each load instruction reads four whole rows;
//   * a row's partial dots are summed over its 16 lanes by a DPP butterfly
//     (every lane gets the same bits); each wave takes its softmax over all
//     its positions at once (max, then 2^(s - max) and p.V), sums its four
//     row slots with lane-swap instructions, and the 8 waves' states are
//     merged in wave order at the end.
// The cache rows read are those below L - 1 (written by earlier steps), so
// the row being appended is never read while it is written.
#pragma once

#include <type_traits>

#include "attn.hpp"
#include "common.hpp"
#include "gemv_mfma.hpp"
#include "params.hpp"

namespace qora {

template <bool F16KV>
__device__ __forceinline__ float4 kv_word_f32(typename std::conditional<F16KV, uint2, float4>::type w) {
    if constexpr (F16KV) return kv_words_f32(w);
    else return w;
}

// c ? a : b per component (a select of the vector objects themselves can be
// lowered through scratch memory)
__device__ __forceinline__ float4 sel4(bool c, float4 a, float4 b) {
    return make_float4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

// The chunked step's exchange for workgroup (head h, column tile j), in two
// halves around a block barrier. chunk_publish (wave 0): the chunk's
// un-normalised state (acc = xr, m = M, l = den) goes to a.part at [h][j]
// and is counted in the head's counter; then lane 0 waits until the head's
// `tiles` states are counted (bounded: past ch_spin polls the step is
// flagged through the range flag and its output is not valid). The states
// are written and read with device-scope atomic stores and loads, and the
// count is raised only once the last store of the wave has returned (an
// exchange whose result the increment depends on), so a counted state is in
// place. Each head's counter has a 128-byte line of its own, and one lane a
// workgroup polls it. chunk_merge (each matrix-core wave, after the
// barrier): the head's states merged in chunk order into M, den and xr of
// the wave's rows (lane * NQ + u).
template <int HD, int NQ>
__device__ __forceinline__ void chunk_publish(const AttnOParams& ap, uint32_t h, uint32_t tile, int lane, float M,
                                              float den, const float (&xr)[NQ]) {
    constexpr uint32_t SR = HD + 2;                     // floats per state: acc[HD], m, l
    float* st = ap.a.part + ((uint64_t)h * ap.g.tiles + tile) * SR;
    uint32_t* count = ap.ch_count + h * kChunkCountStride;
#pragma unroll
    for (int u = 0; u < NQ; ++u)
        __hip_atomic_store(st + lane * NQ + u, xr[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float prev = 0.f;
    if (lane == 0) {
        __hip_atomic_store(st + HD + 1, den, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __hip_atomic_exchange(st + HD, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    uint32_t one = 1u;
    asm volatile("" : "+v"(one) : "v"(prev));
    if (lane == 0) {
        __hip_atomic_fetch_add(count, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t n = 0;
        for (uint32_t it = 0; it < ap.ch_spin; ++it) {
            n = __hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (n >= ap.g.tiles) break;
            __builtin_amdgcn_s_sleep(2);
        }
        fix_flag(ap.g.range_flag, n < ap.g.tiles);
    }
}

template <int HD, int NQ>
__device__ __forceinline__ void chunk_merge(const AttnOParams& ap, uint32_t h, int lane, float& M, float& den,
                                            float (&xr)[NQ]) {
    constexpr uint32_t SR = HD + 2;
    const uint32_t tiles = ap.g.tiles;
    const float* base = ap.a.part + (uint64_t)h * tiles * SR;
    // (m, l) of chunk `lane`, the wave's rows of every chunk (indexes
    // clamped into [0, tiles); weights past `tiles` are zero)
    const uint32_t jl = min((uint32_t)lane, tiles - 1u);
    const float mj = __hip_atomic_load(base + (uint64_t)jl * SR + HD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float lj = __hip_atomic_load(base + (uint64_t)jl * SR + HD + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float ac[kChunkMaxTiles][NQ];
#pragma unroll
    for (uint32_t jj = 0; jj < kChunkMaxTiles; ++jj)
#pragma unroll
        for (int u = 0; u < NQ; ++u)
            ac[jj][u] = __hip_atomic_load(base + (uint64_t)min(jj, tiles - 1u) * SR + lane * NQ + u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    const bool live = (uint32_t)lane < tiles && mj != -INFINITY;
    M = wave_max(live ? mj : -INFINITY);
    const float wl = live ? exp2f(mj - M) : 0.f;
    den = wave_sum(live ? lj * wl : 0.f);
#pragma unroll
    for (int u = 0; u < NQ; ++u) xr[u] = 0.f;
#pragma unroll
    for (uint32_t jj = 0; jj < kChunkMaxTiles; ++jj) {
        const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), (int)jj));
#pragma unroll
        for (int u = 0; u < NQ; ++u) xr[u] = fmaf(ac[jj][u], wj, xr[u]);
    }
}

template <int HD, bool F16KV, int NP, bool CH = false>
__global__ __launch_bounds__(kFusedWaves * kWave) void gemv_q4m_attn_kernel(const void* kc_a, const void* vc_a, const int32_t* pos_a,
                                                                         const long long* qkv_a, const float* ssin_a,
                                                                         uint32_t tg, uint32_t khs, uint32_t cps_a,
                                                                         uint32_t hs_a, AttnOParams ap) {
    constexpr int GW = 1, NW = 4;
    constexpr int KW = HD;                  // one query head per K slice
    constexpr int NKB = KW / 64, NZ = GW * KW / 64;
    constexpr int NQ = HD / 64;             // dim quads per lane
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    static_assert(NP >= 1 && NP <= kFusedMaxPasses, "1 to 8 passes");
    using W = typename std::conditional<F16KV, uint2, float4>::type;
    const GemvParams& p = ap.g;
    const AttnParams& a = ap.a;
    __shared__ __align__(16) float qs[HD];
    __shared__ __align__(16) float kn[HD];
    __shared__ __align__(16) float vn[HD];
    __shared__ __align__(16) float accs[kFusedWaves][HD];
    __shared__ float mls[kFusedWaves][2];
    __shared__ __align__(16) uint8_t zl[NW][GW][4][KW];
    __shared__ __align__(16) uint8_t zero16[16];

    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    // Work item of this workgroup. Workgroups go to the 8 XCDs round-robin
    // (blockIdx % 8); item = (blockIdx % 8) * (grid / 8) + blockIdx / 8 gives
    // each XCD consecutive items, i.e. the column tiles of two query heads of
    // one KV head at the model shape, so an XCD's L2 serves one KV head's
    // rows to all of its workgroups.
    // (the leading arguments are preloaded: tg = tiles | groups << 16, khs =
    // KVH | half << 12 | ss_n << 24, the cache's position and head strides)
    const uint32_t tiles = tg & 0xFFFFu, groups = tg >> 16;
    const uint32_t KVH = khs & 0xFFFu, half = (khs >> 12) & 0xFFFu, ss_n = khs >> 24;
    const uint32_t grid = tiles * KVH * groups;
    const uint32_t item = grid % 8u == 0u ? (blockIdx.x % 8u) * (grid / 8u) + blockIdx.x / 8u : blockIdx.x;
    const uint32_t tile = item % tiles;
    const uint32_t h = item / tiles;                   // K slice = query head
    const uint32_t kvh = h / groups;
    const uint32_t qd = KVH * groups * HD, kvd = KVH * HD;
    const uint64_t cps = cps_a, coff = (uint64_t)kvh * hs_a;

    const uint32_t c = (uint32_t)lane % 16, j = (uint32_t)lane / 16;
    // position of pass i: P0 + 32 i + slot (CH: chunk `tile` of 32 NP
    // positions; otherwise every position from 0)
    const uint32_t P0 = CH ? tile * (kFusedPass * (uint32_t)NP) : 0u;
    const uint32_t slot = P0 + 4u * (uint32_t)wave + j;
    const uint8_t* kcache = reinterpret_cast<const uint8_t*>(kc_a);
    const uint8_t* vcache = reinterpret_cast<const uint8_t*>(vc_a);
    constexpr uint32_t EB = F16KV ? 2u : 4u;
    W kr[NP][NQ], vr[NP][NQ];
    auto row_off = [&](uint32_t pos, int u) {
        return ((uint64_t)pos * cps + coff + 64u * (uint32_t)u + 4u * c) * EB;
    };
    auto load_k = [&](int i, uint32_t pos) {
#pragma unroll
        for (int u = 0; u < NQ; ++u) kr[i][u] = *reinterpret_cast<const W*>(kcache + row_off(pos, u));
    };
    auto load_v = [&](int i, uint32_t pos) {
#pragma unroll
        for (int u = 0; u < NQ; ++u) vr[i][u] = *reinterpret_cast<const W*>(vcache + row_off(pos, u));
    };
    // ---- K rows of passes 0 .. NP-2: positions below 32 (NP - 1) <= L - 1,
    // cached rows whose addresses do not depend on the position (CH: every
    // pass waits for the position) ----
    if constexpr (!CH) {
#pragma unroll
        for (int i = 0; i < NP - 1; ++i) load_k(i, kFusedPass * (uint32_t)i + slot);
    }

    const bool qkv_wave = wave >= NW && wave < NW + HD / kWave;
    const uint32_t d = (uint32_t)(t - NW * kWave) % HD;
    const uint32_t pd = rope_partner(d, half);

    // ---- the position, then the last pass's K rows: rows at or past the
    // appended position are not read (address clamped below it, or to row 0
    // when it is 0; those values are replaced or masked below) ----
    int32_t pos_raw = ld_scalar_i32(pos_a);
    // the parameter block's lines, read while the position is in flight (the
    // position's wait covers them)
    kernarg_warm(ap);
    sgpr_pin(pos_raw);
    const uint32_t L = (uint32_t)pos_raw + 1u;
    const uint32_t cur = L - 1u;                       // position appended this step
    const uint32_t plast = kFusedPass * (uint32_t)(NP - 1) + slot;
    // the row read for position x: rows at or past the appended one are not
    // read (their values are replaced from LDS or masked)
    auto rd = [&](uint32_t x) { return cur == 0u ? 0u : min(x, cur - 1u); };
    const uint32_t plast_rd = rd(plast);
    if constexpr (CH) {
#pragma unroll
        for (int i = 0; i < NP; ++i) load_k(i, rd(kFusedPass * (uint32_t)i + slot));
    } else {
        load_k(NP - 1, plast_rd);
    }

    // ---- the q|k|v sums of the head and its RoPE row (waves NW.., one dim
    // per thread), after the K rows and before the V rows: q is ready while
    // the V rows stream in, and the scores need only q and K ----
    long long qa = 0, qb = 0, ka = 0, kb = 0, va = 0;
    float ssp = 0.f, rc = 1.f, rs = 0.f;
    if (qkv_wave) {
        qa = qkv_a[(uint64_t)h * HD + d];
        qb = qkv_a[(uint64_t)h * HD + pd];
        ka = qkv_a[qd + (uint64_t)kvh * HD + d];
        kb = qkv_a[qd + (uint64_t)kvh * HD + pd];
        va = qkv_a[qd + kvd + (uint64_t)kvh * HD + d];
        ssp = ssin_a[min((uint32_t)lane, ss_n - 1u)];
    }

    // ---- V rows of every pass ----
    if constexpr (CH) {
#pragma unroll
        for (int i = 0; i < NP; ++i) load_v(i, rd(kFusedPass * (uint32_t)i + slot));
    } else {
#pragma unroll
        for (int i = 0; i < NP - 1; ++i) load_v(i, kFusedPass * (uint32_t)i + slot);
        load_v(NP - 1, plast_rd);
    }

    // ---- the matrix-core waves' scales and weights. Waves NW.. issue the
    // same loads as wave - NW (the lines are already in flight): every wave
    // then has the same loads outstanding after its V rows, so its first use
    // of the rows waits for the rows alone, not for these ----
    // ---- the RoPE row of the appended position: its table pointers come
    // from the parameter block, so these loads follow the rows ----
    if (qkv_wave && a.use_rope && d < 2 * half) {
        const uint32_t td = d < half ? d : d - half;
        rc = a.rope_cos[(uint64_t)cur * half + td];
        rs = a.rope_sin[(uint64_t)cur * half + td];
    }

    uint4 wq[GW][NKB];
    uint32_t sw[(NZ + 1) / 2];
    int esg[GW];
    const uint32_t mwave = (uint32_t)wave % NW;
    gemv_q4m_load_scales<GW, NZ>(p.ts, p.tes, (uint64_t)item * NW + mwave, lane, sw, esg);
    gemv_q4m_load_weights<GW, NKB>(p.tw, (uint64_t)item * NW + mwave, lane, wq);
    GemvOut<GW> out{};
    if (wave < NW) out = gemv_q4m_out<GW>(p, tile, wave);
    __builtin_amdgcn_sched_barrier(0);

    if (qkv_wave) {
        // the sums and the RoPE row are waited for here, after the V rows and
        // the weights have been issued
        asm volatile("" : "+v"(qa), "+v"(qb), "+v"(ka), "+v"(kb), "+v"(va), "+v"(ssp), "+v"(rc), "+v"(rs));
        // the q|k|v GEMV ran on x * gamma; its RMSNorm factor is applied here
        const float inv = 1.0f / sqrtf(wave_sum(lane < (int)ss_n ? ssp : 0.f) / (float)a.norm_n + 1e-6f);
        const bool rot = a.use_rope != 0 && d < 2 * half;
        auto rotate = [&](long long x, long long y) {
            const float u = inv * from_fixed(x), v = inv * from_fixed(y);
            return rot ? (d < half ? u * rc - v * rs : u * rc + v * rs) : u;
        };
        qs[d] = rotate(qa, qb);
        float kv = rotate(ka, kb);
        float vv = inv * from_fixed(va);
        const bool owner = tile == 0 && h % groups == 0;
        const uint64_t idx = (uint64_t)cur * cps + coff + d;
        if constexpr (F16KV) {
            const uint16_t kh = f2h(kv), vh = f2h(vv);
            if (owner) {
                reinterpret_cast<uint16_t*>(a.kc)[idx] = kh;
                reinterpret_cast<uint16_t*>(a.vc)[idx] = vh;
            }
            kv = h2f(kh);   // the stored values, as later steps read them
            vv = h2f(vh);
        } else if (owner) {
            reinterpret_cast<float*>(a.kc)[idx] = kv;
            reinterpret_cast<float*>(a.vc)[idx] = vv;
        }
        kn[d] = kv;
        vn[d] = vv;
    }
    if (wave == 0 && lane < 4) reinterpret_cast<uint32_t*>(zero16)[lane] = 0u;
    __syncthreads();

    float q[NQ][4];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        const float4 v = *reinterpret_cast<const float4*>(qs + 64 * u + 4 * c);
        q[u][0] = v.x;
        q[u][1] = v.y;
        q[u][2] = v.z;
        q[u][3] = v.w;
    }
    // ---- scores of the lane's positions, in log2 units (scale * log2 e):
    // the weights 2^(s - m) equal e^(s' - m') of the natural-log scores. In
    // the last pass the appended position takes its k row from LDS and the
    // positions past it are masked ----
    const float scale2 = a.scale * 1.4426950408889634f;   // log2(e)
    // pass i holds the appended position / a live one (CH: any pass; else
    // only the last, whose earlier passes lie below the appended position)
    auto is_cur = [&](int i) { return kFusedPass * (uint32_t)i + slot == cur; };
    auto is_live = [&](int i) { return kFusedPass * (uint32_t)i + slot <= cur; };
    float s[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        float dot = 0.f;
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            float4 k = kv_word_f32<F16KV>(kr[i][u]);
            if (CH || i == NP - 1) {
                // selects, not a masked write into the loaded registers
                const float4 kc4 = *reinterpret_cast<const float4*>(kn + 64 * u + 4 * c);
                k = sel4(is_cur(i), kc4, k);
            }
            dot = fmaf(q[u][0], k.x, dot);
            dot = fmaf(q[u][1], k.y, dot);
            dot = fmaf(q[u][2], k.z, dot);
            dot = fmaf(q[u][3], k.w, dot);
        }
        dot = row16_sum(dot) * scale2;
        s[i] = ((!CH && i < NP - 1) || is_live(i)) ? dot : -INFINITY;
    }
    // ---- the wave's softmax over its positions and p.V (a wave with no
    // live position keeps m = -inf, l = 0, p.V = 0) ----
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < NP; ++i) mx = fmaxf(mx, s[i]);
    mx = wave_max(mx);
    const float mref = mx == -INFINITY ? 0.f : mx;
    // the V rows are first needed below: keep their uses after the softmax
    __builtin_amdgcn_sched_barrier(0);
    float sum = 0.f;
    float o[NQ][4];
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[u][e] = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const float p_i = exp2f(s[i] - mref);      // 0 where masked
        sum += p_i;
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            float4 v = kv_word_f32<F16KV>(vr[i][u]);
            if (CH || i == NP - 1) {
                const float4 vc4 = *reinterpret_cast<const float4*>(vn + 64 * u + 4 * c);
                v = sel4(is_cur(i), vc4, v);
                v = sel4(is_live(i), v, make_float4(0.f, 0.f, 0.f, 0.f));   // select: stale bits never reach the sum
            }
            o[u][0] = fmaf(p_i, v.x, o[u][0]);
            o[u][1] = fmaf(p_i, v.y, o[u][1]);
            o[u][2] = fmaf(p_i, v.z, o[u][2]);
            o[u][3] = fmaf(p_i, v.w, o[u][3]);
        }
    }
    // each row slot counted once (its 16 lanes hold the same weights)
    const float l_w = wave_sum(c == 0 ? sum : 0.f);

    // ---- merge: the wave's 4 row slots, then the 8 waves in order ----
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[u][e] = sum_row_slots(o[u][e]);
    if (j == 0) {
#pragma unroll
        for (int u = 0; u < NQ; ++u)
            *reinterpret_cast<float4*>(&accs[wave][64 * u + 4 * c]) = make_float4(o[u][0], o[u][1], o[u][2], o[u][3]);
    }
    if (lane == 0) {
        mls[wave][0] = mx;
        mls[wave][1] = l_w;
    }
    __syncthreads();
    if (wave >= NW) {
        // the accumulator this launch clears (the next GEMV's), while the
        // matrix-core waves run their pass
        if (p.zero_ptr) {
            const uint32_t tq = (uint32_t)(t - NW * kWave), nq = (kFusedWaves - NW) * kWave;
            for (uint32_t i = blockIdx.x * nq + tq; i < p.zero_n; i += gridDim.x * nq) p.zero_ptr[i] = 0;
        }
        if constexpr (!CH) return;
    }
    // ---- each matrix-core wave merges the 8 waves' states for the rows its
    // lanes quantise (lane l: rows l * NQ + u), in wave order ----
    float M = mls[0][0];
#pragma unroll
    for (int w = 1; w < kFusedWaves; ++w) M = fmaxf(M, mls[w][0]);
    float den = 0.f;
    float xr[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) xr[u] = 0.f;
#pragma unroll
    for (int w = 0; w < kFusedWaves; ++w) {
        const float sc = mls[w][0] == -INFINITY ? 0.f : exp2f(mls[w][0] - M);
        den = fmaf(mls[w][1], sc, den);
#pragma unroll
        for (int u = 0; u < NQ; ++u) xr[u] = fmaf(accs[w][lane * NQ + u], sc, xr[u]);
    }
    if constexpr (CH) {
        if (wave == 0) chunk_publish<HD, NQ>(ap, h, tile, lane, M, den, xr);
        __syncthreads();                               // the head's states are counted
        if (wave >= NW) return;
        chunk_merge<HD, NQ>(ap, h, lane, M, den, xr);
    }
    float xm = 0.f;
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
        xr[u] = xr[u] / den;
        xm = fmaxf(xm, fabsf(xr[u]));
    }
    xm = wave_max(xm);
    gemv_q4m_item<GW, KW>(out, lane, [&xr](int u, uint32_t) { return xr[u]; }, xm, sw, esg, wq, zl[wave], zero16);
}

}  // namespace qora
