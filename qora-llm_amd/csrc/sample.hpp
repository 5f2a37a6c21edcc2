// On-device sampling: the penalties and sample_token_top_k of generate.rs
// (apply_repetition_penalty 64-70, apply_presence_penalty 80-91,
// sample_token_top_k 345-395, Rng 38-61) on the step's logits, so a sampled
// decode step returns a token instead of the 513 KB logits vector.
//
// 1. The penalties: for each distinct history token, the repetition penalty
//    once per occurrence in the last 64 tokens (x / p for x > 0, else x * p,
//    in sequence) and then the presence penalty once if the token occurs
//    anywhere. top_k 1..64 applies them as the first kernel reads the logits;
//    the full-sort path writes a penalised copy (smp_copy_kernel +
//    smp_penalty_kernel).
// 2. smp_block_topk_kernel: each block keeps the best kSmpKeep of its 2048
//    (value, index) keys. Keys order by value descending, then index
//    ascending: the order of the reference's stable sort_by on partial_cmp.
//    NaN ranks last. Each wave sorts runs of 64 keys, one key per lane, with
//    cross-lane exchanges (a bitonic network in registers), and sorted runs
//    are merged pairwise keeping the 64 smallest keys (smp_wave_merge_low).
// 3. smp_final_kernel: one block merges the blocks' sorted candidate runs the
//    same way down to the best 64; the softmax terms of the top k are computed
//    one per lane, and one thread runs the reference's sums in the reference's
//    order (softmax normaliser, nucleus cut-off, one xorshift64 draw, linear
//    scan). Greedy (temperature <= 0) takes the first candidate: the
//    first-max rule.
// The keys are distinct (the index is in the low word), so any correct
// sorting network yields the same order.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace qora {

constexpr uint32_t kSmpBlock = 2048;    // logits per block in the first pass
constexpr uint32_t kSmpKeep = 64;       // candidates kept per block (top_k <= kSmpKeep)
constexpr uint32_t kSmpFinal = 4096;    // candidate keys merged by the final block (64 runs of 64)
constexpr uint32_t kSmpTopkThreads = 512;    // 8 waves: 4 runs of 64 keys each
constexpr uint32_t kSmpFinalThreads = 1024;  // 16 waves: two merges each in the first round
constexpr uint32_t kSmpSortMax = 1u << 22;   // keys of the full-sort path (vocabularies up to 4M)

// Orderable key: ascending key = value descending, then index ascending.
__device__ __forceinline__ unsigned long long smp_key(float v, uint32_t idx) {
    uint32_t b = __float_as_uint(v);
    if (v != v) b = 0xFF800000u;                       // NaN ranks as -inf, after every number
    if (v == 0.0f) b = 0u;                             // -0 == +0: the index decides, as in a stable sort
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);   // ascending with the value
    return ((unsigned long long)(~ord) << 32) | idx;
}
__device__ __forceinline__ float smp_key_value(unsigned long long k) {
    const uint32_t ord = ~(uint32_t)(k >> 32);
    const uint32_t b = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    return __uint_as_float(b);
}

// In-place ascending bitonic sort of n (power of two) keys in LDS by 256 threads.
template <uint32_t N>
__device__ __forceinline__ void smp_bitonic(unsigned long long* keys) {
    for (uint32_t size = 2; size <= N; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (uint32_t i = threadIdx.x; i < N / 2; i += 256) {
                const uint32_t lo = 2 * i - (i & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool up = (lo & size) == 0;
                const unsigned long long a = keys[lo], b = keys[hi];
                if ((a > b) == up) {
                    keys[lo] = b;
                    keys[hi] = a;
                }
            }
        }
    }
    __syncthreads();
}

// A word from lane ^ m (m a power of two below 64, a constant once the
// caller's loops are unrolled): DPP lane moves inside the VALU for 1, 2, 4
// and 8 (quad permutes; a row rotate by 8; rows shifted by 4 either way and
// the lane's direction selected), ds_swizzle for 16, ds_bpermute only for 32.
// (row_shl:n gives lane i the value of lane i + n, row_shr:n of lane i - n.)
__device__ __forceinline__ uint32_t smp_xor_lane(uint32_t x, uint32_t m) {
    const int xi = (int)x;
    switch (m) {
    case 1: return (uint32_t)__builtin_amdgcn_mov_dpp(xi, 0xB1, 0xF, 0xF, false);    // quad_perm [1,0,3,2]
    case 2: return (uint32_t)__builtin_amdgcn_mov_dpp(xi, 0x4E, 0xF, 0xF, false);    // quad_perm [2,3,0,1]
    case 4: {
        const int up = __builtin_amdgcn_mov_dpp(xi, 0x104, 0xF, 0xF, false);        // row_shl:4
        const int dn = __builtin_amdgcn_mov_dpp(xi, 0x114, 0xF, 0xF, false);        // row_shr:4
        return (uint32_t)((threadIdx.x & 4u) ? dn : up);
    }
    case 8: return (uint32_t)__builtin_amdgcn_mov_dpp(xi, 0x128, 0xF, 0xF, false);   // row_ror:8
    case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle(xi, (16 << 10) | 0x1F);    // xor 16 in 32-lane halves
    default: return (uint32_t)__shfl_xor(xi, (int)m, kWave);
    }
}

// One 64-bit key per lane, exchanged with lane ^ m.
__device__ __forceinline__ unsigned long long smp_shfl_xor(unsigned long long v, uint32_t m) {
    const uint32_t lo = smp_xor_lane((uint32_t)v, m), hi = smp_xor_lane((uint32_t)(v >> 32), m);
    return ((unsigned long long)hi << 32) | lo;
}

// The wave's 64 keys (one per lane) sorted ascending in lane order: a
// bitonic network whose exchanges are cross-lane shuffles (no LDS round
// trip, no barrier). Lane i keeps the smaller key when it is the lower lane
// of an ascending block or the upper lane of a descending one.
__device__ __forceinline__ unsigned long long smp_wave_sort(unsigned long long v) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (uint32_t size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            const unsigned long long o = smp_shfl_xor(v, stride);
            const bool keep_min = ((lane & stride) == 0) == ((lane & size) == 0);
            // the keys differ (equal ones are interchangeable), so the lane
            // takes its partner's key exactly when that one belongs here
            v = (o < v) == keep_min ? o : v;
        }
    }
    return v;
}

// The 64 smallest keys of two ascending runs a and b, ascending (lane i
// passes a[i] and b[63 - i]): a followed by b reversed is bitonic, so
// min(a[i], b[63 - i]) holds the 64 smallest as a bitonic sequence, which
// the half-cleaners of strides 32 .. 1 sort.
__device__ __forceinline__ unsigned long long smp_wave_merge_low(unsigned long long a, unsigned long long brev) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    unsigned long long v = brev < a ? brev : a;
#pragma unroll
    for (uint32_t stride = 32; stride > 0; stride >>= 1) {
        const unsigned long long o = smp_shfl_xor(v, stride);
        v = (o < v) == ((lane & stride) == 0) ? o : v;
    }
    return v;
}

// Runs [0, n) of 64 ascending keys in runs[src] merged pairwise (run 2j with
// 2j + 1 into run j of the other buffer, keeping the 64 smallest) until one
// is left, by the block's NWV waves; returns the buffer that holds it.
template <uint32_t N, uint32_t NWV>
__device__ __forceinline__ uint32_t smp_merge_runs(unsigned long long (*runs)[N], uint32_t n, uint32_t src) {
    const uint32_t lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    for (; n > 1; n >>= 1) {
        __syncthreads();
        for (uint32_t j = wave; j < n / 2; j += NWV) {
            const unsigned long long a = runs[src][(2 * j) * 64 + lane];
            const unsigned long long b = runs[src][(2 * j + 1) * 64 + 63 - lane];
            runs[src ^ 1][j * 64 + lane] = smp_wave_merge_low(a, b);
        }
        src ^= 1;
    }
    __syncthreads();
    return src;
}

// The draw's results: the state and the token in device memory, the token
// also as the next decode step's input when asked, and in mapped host memory
// the state and then, after a system-scope fence, the token (the host reads
// the token as soon as it appears, without waiting for the stream).
__device__ __forceinline__ void smp_publish(const SampleParams& p, uint32_t token, unsigned long long state) {
    *p.rng = state;
    *p.token_out = (int32_t)token;
    if (p.dev_token) *p.dev_token = (int32_t)token;
    if (p.host_out) {
        p.host_out[2] = (int32_t)(uint32_t)state;
        p.host_out[3] = (int32_t)(uint32_t)(state >> 32);
        __threadfence_system();
        __hip_atomic_store(p.host_out, (int32_t)token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// One penalty entry applied to x (smp_penalty_kernel's arithmetic).
__device__ __forceinline__ float smp_penalise(const SampleParams& p, const SamplePenalty& e, float x) {
    for (uint32_t r = 0; r < e.rep_count; ++r) x = x > 0.0f ? x / p.repetition : x * p.repetition;
    if (e.seen) x -= p.presence;
    return x;
}

__global__ __launch_bounds__(256) void smp_copy_kernel(const float* in, float* out, uint32_t n) {
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) out[i] = in[i];
}

__global__ __launch_bounds__(256) void smp_penalty_kernel(SampleParams p) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= p.n_pen) return;
    const SamplePenalty e = p.pen[i];
    p.work[e.token] = smp_penalise(p, e, p.work[e.token]);
}

__global__ __launch_bounds__(kSmpTopkThreads) void smp_block_topk_kernel(SampleParams p) {
    constexpr uint32_t NWV = kSmpTopkThreads / kWave;
    static_assert(kSmpKeep == 64 && kSmpBlock % (NWV * 64) == 0, "64-key runs, NWV waves");
    constexpr uint32_t NR = kSmpBlock / 64, RPW = NR / NWV;   // runs, runs per wave
    __shared__ unsigned long long runs[2][kSmpBlock];
    const uint32_t lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const uint32_t base = blockIdx.x * kSmpBlock;
    // every load of the wave's runs first (the logits themselves), the
    // penalties of the block's tokens applied through LDS, then each run
    // sorted across the lanes
    float x[RPW];
#pragma unroll
    for (uint32_t q = 0; q < RPW; ++q) x[q] = p.logits[min(base + (wave + NWV * q) * 64 + lane, p.vocab - 1)];
    if (p.n_pen) {
        float* xs = reinterpret_cast<float*>(runs[1]);
#pragma unroll
        for (uint32_t q = 0; q < RPW; ++q) xs[(wave + NWV * q) * 64 + lane] = x[q];
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < p.n_pen; j += kSmpTopkThreads) {
            const SamplePenalty e = p.pen[j];
            if (e.token >= base && e.token - base < kSmpBlock) xs[e.token - base] = smp_penalise(p, e, xs[e.token - base]);
        }
        __syncthreads();
#pragma unroll
        for (uint32_t q = 0; q < RPW; ++q) x[q] = xs[(wave + NWV * q) * 64 + lane];
        __syncthreads();   // runs[1] is the merge buffer below
    }
    unsigned long long v[RPW];
#pragma unroll
    for (uint32_t q = 0; q < RPW; ++q) {
        const uint32_t i = base + (wave + NWV * q) * 64 + lane;
        v[q] = i < p.vocab ? smp_key(x[q], i) : ~0ull;
    }
#pragma unroll
    for (uint32_t q = 0; q < RPW; ++q) runs[0][(wave + NWV * q) * 64 + lane] = smp_wave_sort(v[q]);
    const uint32_t src = smp_merge_runs<kSmpBlock, NWV>(runs, NR, 0);
    if (wave == 0) p.cand[blockIdx.x * kSmpKeep + lane] = runs[src][lane];
}

__global__ __launch_bounds__(kSmpFinalThreads) void smp_final_kernel(SampleParams p) {
    static_assert(kSmpFinal % 64 == 0 && kSmpKeep == 64, "64-key runs");
    __shared__ unsigned long long runs[2][kSmpFinal];
    __shared__ float prob[kSmpKeep];
    __shared__ float s_inv;
    // the blocks' candidate runs (each ascending), then runs of ~0 padding
    const uint32_t nc = p.blocks * kSmpKeep;
    for (uint32_t j = threadIdx.x; j < kSmpFinal; j += kSmpFinalThreads) runs[0][j] = j < nc ? p.cand[j] : ~0ull;
    const uint32_t src = smp_merge_runs<kSmpFinal, kSmpFinalThreads / kWave>(runs, kSmpFinal / 64, 0);
    const unsigned long long* keys = runs[src];
    const uint32_t k = min(p.top_k, min(p.vocab, kSmpKeep));
    const float inv_temp = p.temperature > 0.0f ? 1.0f / p.temperature : 0.0f;
    // the softmax terms of the top k (generate.rs:360-366), one per lane of
    // wave 0, each the expression the reference evaluates for it
    if (p.temperature > 0.0f && threadIdx.x < k)
        prob[threadIdx.x] = expf((smp_key_value(keys[threadIdx.x]) - smp_key_value(keys[0])) * inv_temp);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        if (p.temperature > 0.0f)
            for (uint32_t i = 0; i < k; ++i) sum += prob[i];
        s_inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    if (p.temperature > 0.0f && threadIdx.x < k && s_inv > 0.0f) prob[threadIdx.x] *= s_inv;
    __syncthreads();
    if (threadIdx.x != 0) return;
    uint32_t token = (uint32_t)keys[0];
    unsigned long long state = p.rng_in;
    if (p.temperature > 0.0f) {
        // softmax over the top k (generate.rs:360-370): the terms and their
        // normalised values are in prob[]; the sum above ran in index order
        if (s_inv > 0.0f) {
            // nucleus cut-off (generate.rs:372-380)
            float cum = 0.0f;
            uint32_t cutoff = k;
            for (uint32_t i = 0; i < k; ++i) {
                cum += prob[i];
                if (cum >= p.top_p) {
                    cutoff = i + 1;
                    break;
                }
            }
            float total = 0.0f;
            for (uint32_t i = 0; i < cutoff; ++i) total += prob[i];
            if (total > 0.0f) {
                // one xorshift64 draw (Rng::next_f32, generate.rs:54-60) and the scan (382-393)
                state ^= state << 13;
                state ^= state >> 7;
                state ^= state << 17;
                const float rand_val = (float)(uint32_t)(state >> 40) / 16777216.0f * total;
                float acc = 0.0f;
                bool hit = false;
                for (uint32_t i = 0; i < cutoff; ++i) {
                    acc += prob[i];
                    if (acc >= rand_val) {
                        token = (uint32_t)keys[i];
                        hit = true;
                        break;
                    }
                }
                if (!hit) token = (uint32_t)keys[0];
            }
        }
    }
    smp_publish(p, token, state);
}

// ---------------------------------------------------------------------------
// Full-sort path: every (value, index) key in the reference's stable order.
// 1. smp_block_sort_kernel: each block bitonic-sorts its 2048 keys and writes
//    them all (keys past the vocabulary are ~0, which sort last);
// 2. smp_merge_kernel, once per doubling of the run length: key i of a run
//    lands at its rank in the run it pairs with (a binary search), so the
//    merged run is in order; the ~0 padding ties break by run (stable);
// 3. smp_probs_kernel: e^((l - max) / temperature) of the first k keys, each
//    computed once by the same expression the scan would use;
// 4. smp_scan_kernel: sample_token_top_k's sums, nucleus cut-off, draw and
//    scan over those k values (generate.rs:360-393), the sums in the
//    reference's order on one lane over LDS-staged values, the draw's scan as
//    a parallel search of the running sums (below).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void smp_block_sort_kernel(SampleParams p) {
    __shared__ unsigned long long keys[kSmpBlock];
    const uint32_t base = blockIdx.x * kSmpBlock;
    for (uint32_t j = threadIdx.x; j < kSmpBlock; j += 256) {
        const uint32_t i = base + j;
        keys[j] = i < p.vocab ? smp_key(p.work[i], i) : ~0ull;
    }
    smp_bitonic<kSmpBlock>(keys);
    for (uint32_t j = threadIdx.x; j < kSmpBlock; j += 256) p.sort_a[base + j] = keys[j];
}

// Runs of `run` keys in `in` (n keys, n a multiple of 2 run) merged in pairs into `out`.
__global__ __launch_bounds__(256) void smp_merge_kernel(const unsigned long long* in, unsigned long long* out,
                                                        uint32_t n, uint32_t run) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const uint32_t r = i / run, base = (r & ~1u) * run;
    const bool first = (r & 1u) == 0u;
    const unsigned long long key = in[i];
    const unsigned long long* other = in + (first ? base + run : base);
    // rank among the other run: keys below (first run) or not above (second
    // run), so equal keys keep their run order
    uint32_t lo = 0, hi = run;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        const bool before = first ? other[mid] < key : other[mid] <= key;
        if (before) lo = mid + 1;
        else hi = mid;
    }
    const uint32_t own = i - (first ? base : base + run);
    out[base + own + lo] = key;
}

__global__ __launch_bounds__(256) void smp_probs_kernel(SampleParams p, const unsigned long long* sorted, uint32_t k) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= k) return;
    const float inv_temp = 1.0f / p.temperature;
    const float max_logit = smp_key_value(sorted[0]);
    p.probs[i] = expf((smp_key_value(sorted[i]) - max_logit) * inv_temp);
}

// The scan of sample_token_top_k (generate.rs:360-393) over the k sorted
// candidates, bit for bit in the reference's float order. Two sequential
// passes run on lane 0 of wave 0 over values staged in LDS (waves 1..3 load
// the next 4096-value chunk while lane 0 works on the current one, so lane 0
// never waits on global memory):
//   A. sum = e_0 + e_1 + ... (left to right), inv = 1 / sum;
//   B. cum_i = cum_{i-1} + e_i * inv, each written back over e_i, up to the
//      first cum_i >= top_p (the cut-off; every value when none reaches it).
// The reference's `total` over the cut-off is the same left-to-right sum of
// the same rounded products, i.e. the last cum_i of pass B, and its draw
// loop recomputes the same running sums: the token is the first candidate
// i < cut-off with cum_i >= rand_val, found by all 256 threads at once.
constexpr uint32_t kScanChunk = 4096;

__device__ __forceinline__ void smp_scan_stage(const float* src, uint32_t c, uint32_t n, float* dst) {
    for (uint32_t i = threadIdx.x - 64u; i < kScanChunk; i += 192u) {
        const uint32_t j = c * kScanChunk + i;
        dst[i] = j < n ? src[j] : 0.f;
    }
}

// The reference's running fp32 sum over x_0 .. x_{n-1}, s_i = fl(s_{i-1} + x_i)
// from s_{-1} = 0, bit for bit, by all 256 threads. While s stays in one
// binade [2^E, 2^(E+1)) (or below 2^-126), every sum lies on the grid
// u = 2^(E-23) (2^-149 below): s + x rounds to s + RNE(x / u) grid units as
// long as that stays below the binade's end, and RNE(x / u) of a value that
// is not exactly half a unit off the grid does not depend on s. So each
// thread classifies its values against the grid (integer arithmetic on their
// bits), a saturating prefix sum of the units gives every running sum of a
// 4096-value chunk at once, and a block minimum finds the first event: a tie
// (half a unit: the result's parity decides), a sum reaching the binade's end,
// a value that is not a finite number >= 0, or (STOP) a sum >= stop. The sums
// before the event are exact grid values; the event's value is added with one
// fp32 addition, the reference's own operation, and the chunk restarts after
// it. Events are rare: a binade crossing per doubling of the sum, a tie only
// when a value's bits end exactly half a unit off the grid.
// Returns the sum (with STOP: the sum at the first s_i >= stop, and
// *stop_at = i + 1; 0 when no sum reaches it). WRITE: s_i goes to out[i] for
// every i up to the stop (or n).
constexpr uint32_t kExactJ = 16;                       // values per thread per chunk
constexpr uint32_t kExactChunk = 256 * kExactJ;
constexpr uint32_t kExactCap = 1u << 25;               // saturation of the unit sums (above every binade's end)
constexpr uint32_t kExactNone = 0xFFFFFFFFu;

struct SmpExactShared {
    uint32_t wtot[4], wmin[4];
    float s;
    uint32_t base, stop_at, done;
};

__device__ __forceinline__ uint32_t smp_sat_add(uint32_t a, uint32_t b) { return min(a + b, kExactCap); }

// Units of x on the grid 2^eu, rounded to nearest, and whether x is an event
// by itself (exactly half a unit off the grid, not a finite number >= 0).
__device__ __forceinline__ uint32_t smp_grid_units(float x, int eu, bool& ev) {
    // every case computed and selected (no branches: 16 values a thread)
    const uint32_t b = __float_as_uint(x);
    const bool zero = (b & 0x7FFFFFFFu) == 0u;         // +-0
    const bool bad = !zero && b >= 0x7F800000u;        // inf, NaN, or a negative value
    const uint32_t ef = (b >> 23) & 0xFFu;
    const uint32_t mx = ef ? ((b & 0x7FFFFFu) | 0x800000u) : (b & 0x7FFFFFu);
    const int sh = (ef ? (int)ef - 150 : -149) - eu;   // x = mx * 2^(eu + sh)
    // sh >= 0: whole units (at least 2^31 beyond 7: saturated)
    const uint32_t up = sh >= 8 ? kExactCap : min(mx << (uint32_t)min(max(sh, 0), 7), kExactCap);
    // sh < 0: rounded to nearest; below a quarter unit (d > 25) nothing, and no tie
    const uint32_t d = (uint32_t)min(max(-sh, 1), 26);
    const uint32_t rem = mx & ((1u << d) - 1u), half = 1u << (d - 1u);
    const uint32_t dn = (mx >> d) + (rem > half ? 1u : 0u);
    ev = bad || (!zero && sh < 0 && rem == half);
    return zero || bad ? 0u : (sh >= 0 ? up : dn);
}

template <bool STOP, bool WRITE, typename Val>
__device__ float smp_exact_sum(uint32_t n, Val val, float stop, float* out, uint32_t* stop_at, SmpExactShared& sh) {
    const uint32_t t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
    if (t == 0) {
        sh.s = 0.0f;
        sh.base = 0;
        sh.stop_at = 0;
        sh.done = 0;
    }
    __syncthreads();
    // windows of 4096 values, each loaded once (the next one in flight while
    // this one is worked on); an event restarts within the window, the values
    // before the restart masked out
    // (loads are unconditional, at an index clamped into the values, and the
    // values past n then replaced: no branch per value)
    float xn[kExactJ];
#pragma unroll
    for (uint32_t j = 0; j < kExactJ; ++j) {
        const uint32_t in = t * kExactJ + j;
        const float v = val(min(in, n - 1u));
        xn[j] = in < n ? v : 0.0f;
    }
    for (uint32_t w0 = 0; w0 < n; w0 += kExactChunk) {
      const uint32_t i0 = w0 + t * kExactJ;
      float x[kExactJ];
#pragma unroll
      for (uint32_t j = 0; j < kExactJ; ++j) {
          x[j] = xn[j];
          const uint32_t in = i0 + kExactChunk + j;
          const float v = val(min(in, n - 1u));
          xn[j] = in < n ? v : 0.0f;
      }
      for (;;) {
        const float s = sh.s;
        const uint32_t base = sh.base;
        if (sh.done || base >= n || base >= w0 + kExactChunk) break;
        // the binade of s: grid 2^eu, s = M units, its end at `bound` units
        const uint32_t sb = __float_as_uint(s);
        const int eu = sb < 0x00800000u ? -149 : (int)(sb >> 23) - 150;
        const uint32_t M = sb < 0x00800000u ? sb : ((sb & 0x7FFFFFu) | 0x800000u);
        const uint32_t bound = sb < 0x00800000u ? (1u << 23) : (1u << 24);
        uint32_t loc[kExactJ];
        uint32_t evm = 0;                              // bit j: value j is an event by itself
        uint32_t acc = 0;
        // bit j: value j lies in [base, n)
        const uint32_t lo = (uint32_t)min(max((int)(base - i0), 0), (int)kExactJ);
        const uint32_t hi = (uint32_t)min(max((int)(n - i0), 0), (int)kExactJ);
        const uint32_t liveb = ((1u << hi) - 1u) & ~((1u << lo) - 1u);
#pragma unroll
        for (uint32_t j = 0; j < kExactJ; ++j) {
            const bool live = (liveb >> j) & 1u;
            bool ev;
            const uint32_t r = smp_grid_units(live ? x[j] : 0.0f, eu, ev);
            evm |= (ev ? 1u : 0u) << j;
            acc = smp_sat_add(acc, r);
            loc[j] = acc;
        }
        // exclusive prefix of the threads' totals (saturating)
        uint32_t inc = acc;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)inc, (unsigned)d, kWave);
            if (lane >= (uint32_t)d) inc = smp_sat_add(inc, o);
        }
        // the lane's exclusive prefix is the previous lane's inclusive one (not
        // inc - acc: a saturated inc has lost it)
        const uint32_t exw = (uint32_t)__shfl_up((int)inc, 1u, kWave);
        if (lane == kWave - 1) sh.wtot[wave] = inc;
        __syncthreads();
        uint32_t prev = 0;
        for (uint32_t w = 0; w < wave; ++w) prev = smp_sat_add(prev, sh.wtot[w]);
        const uint32_t excl = smp_sat_add(prev, lane ? exw : 0u);
        // this thread's first event (chunk index), then the block's
        uint32_t eb = evm;
#pragma unroll
        for (uint32_t j = 0; j < kExactJ; ++j) {
            const uint32_t P = smp_sat_add(excl, loc[j]);
            bool e = M + P >= bound;
            if (STOP) e = e || ldexpf((float)(M + P), eu) >= stop;
            eb |= (e ? 1u : 0u) << j;
        }
        eb &= liveb;
        uint32_t fe = eb ? t * kExactJ + (uint32_t)__builtin_ctz(eb) : kExactNone;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) fe = min(fe, (uint32_t)__shfl_xor((int)fe, off, kWave));
        if (lane == 0) sh.wmin[wave] = fe;
        __syncthreads();
        const uint32_t first = min(min(sh.wmin[0], sh.wmin[1]), min(sh.wmin[2], sh.wmin[3]));
        // the exact sums before the event (or the chunk's end)
        if (WRITE) {
#pragma unroll
            for (uint32_t j = 0; j < kExactJ; ++j)
                if (((liveb >> j) & 1u) && t * kExactJ + j < first)
                    out[i0 + j] = ldexpf((float)(M + smp_sat_add(excl, loc[j])), eu);
        }
        if (first == kExactNone) {
            if (t == 0) {
                uint32_t tot = 0;
                for (uint32_t w = 0; w < 4; ++w) tot = smp_sat_add(tot, sh.wtot[w]);
                sh.s = ldexpf((float)(M + tot), eu);
                sh.base = min(n, w0 + kExactChunk);
            }
        } else if (t == first / kExactJ) {
            // the event's value, added to the exact sum before it
            const uint32_t j = first % kExactJ;
            float xe = x[0];
            uint32_t before = excl;
#pragma unroll
            for (uint32_t q = 0; q < kExactJ; ++q)
                if (q == j) xe = x[q];
#pragma unroll
            for (uint32_t q = 0; q < kExactJ; ++q)
                if (q + 1 == j) before = smp_sat_add(excl, loc[q]);
            const float sn = __fadd_rn(ldexpf((float)(M + before), eu), xe);
            const uint32_t gi = w0 + first;
            if (WRITE) out[gi] = sn;
            sh.s = sn;
            sh.base = gi + 1;
            if (STOP && sn >= stop) {
                sh.stop_at = gi + 1;
                sh.done = 1;
            } else if (!(sn <= 3.402823466e38f)) {
                sh.done = 1;                           // NaN (or inf): every later sum stays so
            }
        }
        __syncthreads();
      }
      if (sh.done) break;
    }
    const float r = sh.s;
    if (STOP) *stop_at = sh.stop_at;
    __syncthreads();                                   // sh is reused by the next call
    return r;
}

__global__ __launch_bounds__(256) void smp_scan_kernel(SampleParams p, const unsigned long long* sorted, uint32_t k) {
    __shared__ __align__(16) float buf[2][kScanChunk];
    __shared__ SmpExactShared sx;
    __shared__ float s_val[2];
    __shared__ uint32_t s_hit[4];
    const uint32_t t = threadIdx.x;
    uint32_t token = (uint32_t)sorted[0];
    unsigned long long state = p.rng_in;
    if (p.temperature > 0.0f) {
        const float* probs = p.probs;
        const float sum = smp_exact_sum<false, false>(k, [probs](uint32_t i) { return probs[i]; }, 0.0f, nullptr,
                                                      nullptr, sx);
        if (t == 0) s_val[0] = sum;
        __syncthreads();
        if (s_val[0] > 0.0f) {
            const float inv = 1.0f / s_val[0];
            // each probability is e * inv, rounded, then added (never one fused
            // multiply-add), as the reference scales the vector before summing
            uint32_t stop = 0;
            const float cum = smp_exact_sum<true, true>(
                k, [probs, inv](uint32_t i) { return __fmul_rn(probs[i], inv); }, p.top_p, p.probs, &stop, sx);
            const uint32_t cutoff = stop ? stop : k;
            if (t == 0) s_val[1] = cum;   // total over the cut-off
            __syncthreads();
            const float total = s_val[1];
            if (total > 0.0f) {
                state ^= state << 13;
                state ^= state >> 7;
                state ^= state << 17;
                const float rand_val = (float)(uint32_t)(state >> 40) / 16777216.0f * total;
                // C: first i < cutoff with cum_i >= rand_val, a staged chunk at a
                // time, every thread testing its values of the chunk (the cum_i
                // are this block's own stores, ordered by the barriers)
                const uint32_t nch = (cutoff + kScanChunk - 1) / kScanChunk;
                if (t >= 64) smp_scan_stage(p.probs, 0, cutoff, buf[0]);
                __syncthreads();
                uint32_t first = 0xFFFFFFFFu;
                for (uint32_t c = 0; c < nch; ++c) {
                    if (t >= 64 && c + 1 < nch) smp_scan_stage(p.probs, c + 1, cutoff, buf[(c + 1) & 1u]);
                    const float* b = buf[c & 1u];
                    const uint32_t i0 = c * kScanChunk, cnt = min(kScanChunk, cutoff - i0);
                    uint32_t f = 0xFFFFFFFFu;
                    for (uint32_t j = t; j < cnt; j += 256)
                        if (b[j] >= rand_val) {
                            f = i0 + j;
                            break;
                        }
#pragma unroll
                    for (int off = 32; off >= 1; off >>= 1) f = min(f, (uint32_t)__shfl_xor((int)f, off, kWave));
                    if ((t & 63u) == 0) s_hit[t / 64] = f;
                    __syncthreads();
                    first = min(min(s_hit[0], s_hit[1]), min(s_hit[2], s_hit[3]));
                    __syncthreads();   // s_hit is rewritten next chunk
                    if (first != 0xFFFFFFFFu) break;
                }
                if (first != 0xFFFFFFFFu) token = (uint32_t)sorted[first];
            }
        }
    }
    if (t == 0) smp_publish(p, token, state);
}

}  // namespace qora
