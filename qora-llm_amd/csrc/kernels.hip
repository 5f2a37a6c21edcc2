// Kernel instantiations and launch helpers (gfx950).
#include "launch.hpp"
#include "gemv.hpp"
#include "gemv_mfma.hpp"
#include "lmhead_mfma.hpp"
#include "attn.hpp"
#include "attn_o.hpp"
#include "prefill.hpp"
#include "sample.hpp"

#include <algorithm>
#include <cstring>
#include <cstdlib>

namespace qora {

const char* tuning_env(const char* name) {
    const char* on = std::getenv("QORA_HIP_TUNING");
    if (!on || std::strcmp(on, "1") != 0) return nullptr;
    const char* v = std::getenv(name);
    return (v && *v) ? v : nullptr;
}

static int env_int(const char* name, int dflt) {
    const char* v = tuning_env(name);
    return v ? std::atoi(v) : dflt;
}

bool plan_gemv(int fmt, uint32_t k, const uint32_t* seg_groups, int nseg, bool paired, int cus,
               GemvPlan* plan, uint32_t row_align) {
    if (k == 0 || nseg < 1 || nseg > 3 || row_align == 0) return false;
    if (paired && (nseg != 2 || seg_groups[0] != seg_groups[1])) return false;
    GemvPlan pl;
    pl.gt = paired ? 16 : 8;
    const int forced_gt = env_int("QORA_GEMV_GT", 0);
    if (!paired && (forced_gt == 8 || forced_gt == 16)) pl.gt = forced_gt;
    if (paired) {
        pl.tiles = (seg_groups[0] + pl.gt / 2 - 1) / (pl.gt / 2);
    } else {
        pl.tiles = 0;
        for (int i = 0; i < nseg; ++i) pl.tiles += (seg_groups[i] + pl.gt - 1) / pl.gt;
    }
    const uint32_t rl = 256 / pl.gt;
    const int max_rpl = (fmt == FMT_Q4) ? 16 : 8;
    const uint32_t target = (uint32_t)std::max(1, cus) * 2;   // ~2 workgroups per CU
    const uint32_t s_des = std::max(1u, (target + pl.tiles / 2) / pl.tiles);
    const uint32_t kr_des = (k + s_des - 1) / s_des;
    const uint32_t rpl_des = std::max(1u, (kr_des + rl - 1) / rl);
    int rpl = 1;
    while (rpl < max_rpl && (uint32_t)rpl * 3 / 2 < rpl_des) rpl *= 2;   // nearest power of two
    const int forced_rpl = env_int("QORA_GEMV_RPL", 0);
    if ((forced_rpl == 1 || forced_rpl == 2 || forced_rpl == 4 || forced_rpl == 8 || forced_rpl == 16) &&
        forced_rpl <= max_rpl)
        rpl = forced_rpl;
    while (rpl < max_rpl && ((rl * (uint32_t)rpl) % row_align) != 0) rpl *= 2;
    // at most kFixMaxTerms split-K terms per accumulator between two reads
    // (the fixed-point range guard, params.hpp)
    while (rpl < max_rpl && (k + rl * (uint32_t)rpl - 1) / (rl * (uint32_t)rpl) > kFixMaxTerms) rpl *= 2;
    if ((rl * (uint32_t)rpl) % row_align != 0) return false;
    pl.rpl = rpl;
    pl.kr = rl * (uint32_t)rpl;
    pl.splits = (k + pl.kr - 1) / pl.kr;
    *plan = pl;
    return true;
}

bool plan_gemv_q4m(uint32_t k, const uint32_t* seg_groups, int nseg, bool paired, int cus, GemvPlan* plan,
                   uint32_t row_align, uint32_t force_kw) {
    if (k == 0 || nseg < 1 || nseg > 3 || row_align == 0) return false;
    if (paired && (nseg != 2 || seg_groups[0] != seg_groups[1])) return false;
    // One group (32 columns) per wave and the deepest K slice that still
    // gives every CU a workgroup: measured on the decode shapes, deeper
    // slices beat wider tiles (fewer workgroups pay the input latency and
    // the atomics, and each streams a longer contiguous block).
    static const uint32_t kws[3] = {256, 128, 64};
    const uint32_t want = (uint32_t)std::max(1, cus);
    const int forced_gw = force_kw ? 1 : env_int("QORA_GEMV_GW", 0);
    const int forced_kw = force_kw ? (int)force_kw : env_int("QORA_GEMV_KW", 0);
    const int gw = (forced_gw == 1 || forced_gw == 2 || forced_gw == 4) ? forced_gw : 1;
    if (forced_kw == 512) {
        // 512-row slices (one group per wave), only when asked for
        if (gw != 1 || row_align > 512 || 512 % row_align != 0) return false;
        GemvPlan pl;
        pl.mfma = 1;
        pl.gw = 1;
        pl.gt = 4;
        pl.rpl = 0;
        if (paired) {
            pl.tiles = (seg_groups[0] + 1) / 2;
        } else {
            pl.tiles = 0;
            for (int i = 0; i < nseg; ++i) pl.tiles += (seg_groups[i] + 3) / 4;
        }
        pl.kr = 512;
        pl.splits = (k + 511) / 512;
        *plan = pl;
        return true;
    }
    GemvPlan best;
    bool have = false;
    for (uint32_t kw : kws) {
        if (forced_kw && kw != (uint32_t)forced_kw) continue;
        if (!(kw % row_align == 0 || row_align % kw == 0)) continue;
        GemvPlan pl;
        pl.mfma = 1;
        pl.gw = gw;
        pl.gt = 4 * gw;
        pl.rpl = 0;
        if (paired) {
            pl.tiles = (seg_groups[0] + 2 * gw - 1) / (2 * gw);
        } else {
            pl.tiles = 0;
            for (int i = 0; i < nseg; ++i) pl.tiles += (seg_groups[i] + pl.gt - 1) / pl.gt;
        }
        pl.kr = kw;
        pl.splits = (k + pl.kr - 1) / pl.kr;
        // an accumulator takes at most kFixMaxTerms split-K terms between two
        // reads (the fixed-point range guard, params.hpp)
        if (pl.splits > kFixMaxTerms) continue;
        if (!have || (best.blocks() < want && pl.blocks() > best.blocks())) {
            best = pl;
            have = true;
        }
        if (best.blocks() >= want) break;
    }
    if (!have) return false;
    *plan = best;
    return true;
}

void apply_plan(const GemvPlan& plan, GemvParams* p) {
    uint32_t t0 = 0, c0 = 0;
    for (int i = 0; i < p->nseg; ++i) {
        p->seg[i].tile0 = p->paired ? 0 : t0;
        p->seg[i].tiles = p->paired ? plan.tiles : (p->seg[i].groups + plan.gt - 1) / plan.gt;
        p->seg[i].col0 = c0;
        t0 += p->seg[i].tiles;
        c0 += p->seg[i].groups * 32u;
    }
    p->tiles = plan.tiles;
    p->splits = plan.splits;
    p->rows_per_split = plan.kr;
    // XCD order for the prologues that read a previous kernel's output (bit
    // = prologue): each XCD's L2 then fetches the inputs of its own K slices
    // only. The plain prologue's input is one small vector; it keeps launch
    // order, which streams its weights a little faster.
    static const int xcd_mask = env_int("QORA_HIP_XCD_ORDER",
                                        (1 << PRO_GAMMA_FIXED) | (1 << PRO_SILU_FIXED) | (1 << PRO_ATTN));
    p->xcd_order = (uint32_t)(xcd_mask >> p->pro) & 1u;
}

template <int FMT, int GT, int PRO, bool TILED>
static hipError_t launch_gemv_pro(const GemvPlan& plan, const GemvParams& p, hipStream_t stream) {
    const dim3 grid(plan.blocks()), block(256);
    // the first loads' arguments ahead of the parameter block (preloaded into
    // scalar registers at wave launch); ss_n | norm_n << 8 in one word
    if (p.ss_n > 0xFFu || p.norm_n >= (1u << 24)) return hipErrorInvalidValue;
    const void* xin = PRO == PRO_PLAIN ? static_cast<const void*>(p.x) : static_cast<const void*>(p.xacc);
    const void* xaux = PRO == PRO_GAMMA_FIXED ? static_cast<const void*>(p.gamma)
                                              : static_cast<const void*>(p.ss_in);
    const uint32_t ss_nn = p.ss_n | (p.norm_n << 8);
#define QORA_GEMV_ARGS p.tw, p.ts, xin, xaux, p.k, p.tiles, p.rows_per_split, ss_nn, p
    switch (plan.rpl) {
    case 1: hipLaunchKernelGGL((gemv_kernel<FMT, GT, 1, PRO, TILED>), grid, block, 0, stream, QORA_GEMV_ARGS); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<FMT, GT, 2, PRO, TILED>), grid, block, 0, stream, QORA_GEMV_ARGS); break;
    case 4: hipLaunchKernelGGL((gemv_kernel<FMT, GT, 4, PRO, TILED>), grid, block, 0, stream, QORA_GEMV_ARGS); break;
    case 8: hipLaunchKernelGGL((gemv_kernel<FMT, GT, 8, PRO, TILED>), grid, block, 0, stream, QORA_GEMV_ARGS); break;
    case 16:
        if constexpr (FMT == FMT_Q4) {
            hipLaunchKernelGGL((gemv_kernel<FMT, GT, 16, PRO, TILED>), grid, block, 0, stream, QORA_GEMV_ARGS);
            break;
        }
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
#undef QORA_GEMV_ARGS
    return hipGetLastError();
}

template <int FMT, int GT>
static hipError_t launch_gemv_gt(const GemvPlan& plan, const GemvParams& p, hipStream_t stream) {
    if (!p.tw) {
        // reference layout: the kernel-level plain GEMV entry points only
        if (p.pro != PRO_PLAIN) return hipErrorInvalidValue;
        return launch_gemv_pro<FMT, GT, PRO_PLAIN, false>(plan, p, stream);
    }
    if constexpr (FMT == FMT_Q4) {
        return hipErrorInvalidValue;   // the Q4 tile layout runs on the matrix cores (launch_q4m_*)
    } else {
        switch (p.pro) {
        case PRO_PLAIN: return launch_gemv_pro<FMT, GT, PRO_PLAIN, true>(plan, p, stream);
        case PRO_GAMMA_FIXED: return launch_gemv_pro<FMT, GT, PRO_GAMMA_FIXED, true>(plan, p, stream);
        case PRO_SILU_FIXED: return launch_gemv_pro<FMT, GT, PRO_SILU_FIXED, true>(plan, p, stream);
        case PRO_ATTN: return launch_gemv_pro<FMT, GT, PRO_ATTN, true>(plan, p, stream);
        default: return hipErrorInvalidValue;
        }
    }
}

template <int GW, int KW, int IPW>
static hipError_t launch_q4m_ipw(const GemvPlan& plan, const GemvParams& p, hipStream_t stream) {
    // 4 matrix-core waves that build their own input rows; the attention
    // merge keeps 4 matrix-core waves + 4 prologue waves
    const dim3 grid(plan.grid()), block(256), block_attn(512);
    // the 4-wave kernel takes the item count (bit 31: XCD order) and
    // ss_n | norm_n << 8 in single argument words
    if (plan.grid() >= 0x80000000u || (p.pro == PRO_SILU_FIXED && (p.ss_n > 0xFFu || p.norm_n >= (1u << 24))))
        return hipErrorInvalidValue;
    switch (p.pro) {
    case PRO_PLAIN:
        hipLaunchKernelGGL((gemv_q4m4_kernel<GW, KW, PRO_PLAIN>), grid, block, 0, stream, p.tw, p.ts, p.tes,
                           static_cast<const void*>(p.x), static_cast<const void*>(nullptr), p.k, p.tiles,
                           plan.grid() | (p.xcd_order ? 0x80000000u : 0u), p.ss_n | (p.norm_n << 8), p);
        break;
    case PRO_GAMMA_FIXED:
        hipLaunchKernelGGL((gemv_q4m4_kernel<GW, KW, PRO_GAMMA_FIXED>), grid, block, 0, stream, p.tw, p.ts, p.tes,
                           static_cast<const void*>(p.xacc), static_cast<const void*>(p.gamma), p.k, p.tiles,
                           plan.grid() | (p.xcd_order ? 0x80000000u : 0u), p.ss_n | (p.norm_n << 8), p);
        break;
    case PRO_SILU_FIXED:
        hipLaunchKernelGGL((gemv_q4m4_kernel<GW, KW, PRO_SILU_FIXED>), grid, block, 0, stream, p.tw, p.ts, p.tes,
                           static_cast<const void*>(p.xacc), static_cast<const void*>(p.ss_in), p.k, p.tiles,
                           plan.grid() | (p.xcd_order ? 0x80000000u : 0u), p.ss_n | (p.norm_n << 8), p);
        break;
    case PRO_ATTN:
        if constexpr (IPW == 1) {
            if (p.head_dim > 0x3FFu || p.groups > 0x3FFu || p.attn_s_max > 0xFFFu) return hipErrorInvalidValue;
            hipLaunchKernelGGL((gemv_q4m_kernel<GW, KW, PRO_ATTN, 1>), grid, block_attn, 0, stream, p.tw, p.ts, p.tes,
                               p.attn_part, p.pos, p.k, p.tiles, plan.grid() | (p.xcd_order ? 0x80000000u : 0u),
                               p.head_dim | (p.groups << 10) | (p.attn_s_max << 20), p);
            break;
        } else {
            return hipErrorInvalidValue;
        }
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int GW, int KW>
static hipError_t launch_q4m_kw(const GemvPlan& plan, const GemvParams& p, hipStream_t stream) {
    if (plan.ipw != 1) return hipErrorInvalidValue;
    return launch_q4m_ipw<GW, KW, 1>(plan, p, stream);
}

template <int GW>
static hipError_t launch_q4m_gw(const GemvPlan& plan, const GemvParams& p, hipStream_t stream) {
    switch (plan.kr) {
    case 64: return launch_q4m_kw<GW, 64>(plan, p, stream);
    case 128: return launch_q4m_kw<GW, 128>(plan, p, stream);
    case 256: return launch_q4m_kw<GW, 256>(plan, p, stream);
    case 512:
        if constexpr (GW == 1) return launch_q4m_kw<1, 512>(plan, p, stream);
        else return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(int fmt, const GemvPlan& plan, const GemvParams& p, hipStream_t stream) {
    if (plan.blocks() == 0) return hipErrorInvalidValue;
    if (plan.mfma) {
        if (plan.ipw != 1 && (p.pro == PRO_ATTN || plan.gw != 1 || plan.kr != 256)) return hipErrorInvalidValue;
        if (fmt != FMT_Q4 || !p.tw || !p.ts || !p.tes) return hipErrorInvalidValue;
        switch (plan.gw) {
        case 1: return launch_q4m_gw<1>(plan, p, stream);
        case 2: return launch_q4m_gw<2>(plan, p, stream);
        case 4: return launch_q4m_gw<4>(plan, p, stream);
        default: return hipErrorInvalidValue;
        }
    }
    if (fmt == FMT_Q4) {
        if (plan.gt == 8) return launch_gemv_gt<FMT_Q4, 8>(plan, p, stream);
        if (plan.gt == 16) return launch_gemv_gt<FMT_Q4, 16>(plan, p, stream);
    } else {
        if (plan.gt == 8) return launch_gemv_gt<FMT_F16, 8>(plan, p, stream);
        if (plan.gt == 16) return launch_gemv_gt<FMT_F16, 16>(plan, p, stream);
    }
    return hipErrorInvalidValue;
}

void gemv_tile_bytes(int fmt, const GemvPlan& plan, uint64_t* w_bytes, uint64_t* s_bytes, uint64_t* e_bytes) {
    if (plan.mfma) {
        const uint64_t waves = (uint64_t)plan.blocks() * 4u;
        const uint64_t nkb = plan.kr / 64u, nz = (uint64_t)plan.gw * plan.kr / 64u;
        *w_bytes = waves * (uint64_t)plan.gw * nkb * 1024u;
        *s_bytes = waves * 64u * nz * 2u;
        *e_bytes = waves * (uint64_t)plan.gw;
        return;
    }
    const uint64_t steps = (uint64_t)plan.blocks() * (uint64_t)plan.rpl;
    *w_bytes = steps * 256u * (fmt == FMT_Q4 ? 16u : 64u);
    *s_bytes = fmt == FMT_Q4 ? steps * 256u * 2u : 0u;
    *e_bytes = 0;
}

hipError_t launch_gemv_tile(int fmt, const GemvPlan& plan, const GemvParams& p, uint8_t* tw, uint16_t* ts,
                            int8_t* te, hipStream_t stream) {
    if (p.k == 0) return hipErrorInvalidValue;
    if (plan.mfma) {
        const uint64_t grid = (uint64_t)plan.blocks() * 4u;
        if (fmt != FMT_Q4 || !ts || !te || grid == 0 || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gemv_q4m_pack_kernel, dim3((uint32_t)grid), dim3(64), 0, stream, p, plan.gw, (int)plan.kr,
                           tw, ts, te);
        return hipGetLastError();
    }
    const uint64_t grid = (uint64_t)plan.blocks() * (uint64_t)plan.rpl;
    if (grid == 0 || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (fmt == FMT_Q4) {
        if (!ts) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gemv_tile_kernel<FMT_Q4>, dim3((uint32_t)grid), dim3(256), 0, stream, p, plan.gt, plan.rpl,
                           tw, ts);
    } else {
        hipLaunchKernelGGL(gemv_tile_kernel<FMT_F16>, dim3((uint32_t)grid), dim3(256), 0, stream, p, plan.gt,
                           plan.rpl, tw, ts);
    }
    return hipGetLastError();
}

// Element i of the token-major rows [len][kvh][hd] sits at ((h * cap + t) * hd + d) of one
// layer's head-major cache [kvh][cap][hd]; TO_CACHE moves rows into the cache, else back out.
template <bool TO_CACHE, bool F16>
__global__ __launch_bounds__(256) void kv_move_kernel(float* rows, void* cache, uint32_t len, uint32_t kvh,
                                                      uint32_t hd, uint64_t cap) {
    const uint64_t row = (uint64_t)kvh * hd, n = (uint64_t)len * row;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t t = i / row;
        const uint32_t r = (uint32_t)(i - t * row);
        const uint32_t h = r / hd, d = r - h * hd;
        const uint64_t o = ((uint64_t)h * cap + t) * hd + d;
        if constexpr (TO_CACHE) {
            if constexpr (F16) ((uint16_t*)cache)[o] = f2h(rows[i]);
            else ((float*)cache)[o] = rows[i];
        } else {
            if constexpr (F16) rows[i] = h2f(((const uint16_t*)cache)[o]);
            else rows[i] = ((const float*)cache)[o];
        }
    }
}

hipError_t launch_kv_move(bool to_cache, bool f16, float* rows, void* cache, uint32_t len, uint32_t kvh, uint32_t hd,
                          uint64_t cap, hipStream_t stream) {
    const uint64_t n = (uint64_t)len * kvh * hd;
    if (n == 0) return hipSuccess;
    if (len > cap || hd == 0) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)std::min<uint64_t>(4096, (n + 255) / 256)), block(256);
    if (to_cache) {
        if (f16) hipLaunchKernelGGL((kv_move_kernel<true, true>), grid, block, 0, stream, rows, cache, len, kvh, hd, cap);
        else hipLaunchKernelGGL((kv_move_kernel<true, false>), grid, block, 0, stream, rows, cache, len, kvh, hd, cap);
    } else {
        if (f16) hipLaunchKernelGGL((kv_move_kernel<false, true>), grid, block, 0, stream, rows, cache, len, kvh, hd, cap);
        else hipLaunchKernelGGL((kv_move_kernel<false, false>), grid, block, 0, stream, rows, cache, len, kvh, hd, cap);
    }
    return hipGetLastError();
}

hipError_t launch_fill_zero(long long* p, uint64_t n, hipStream_t stream) {
    const uint32_t blocks = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(1024, (n + 255) / 256));
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

hipError_t launch_acc_to_f32(const long long* acc, uint32_t n, int paired, float* y, hipStream_t stream) {
    const uint32_t blocks = std::max(1u, std::min(1024u, (n + 255) / 256));
    hipLaunchKernelGGL(acc_to_f32_kernel, dim3(blocks), dim3(256), 0, stream, acc, n, paired, y);
    return hipGetLastError();
}

static constexpr int kRowdotU = 8;

uint32_t rowdot_blocks(uint32_t rows, uint32_t cols, int cus) {
    const uint32_t G = cols / 32;
    const uint32_t rpw = G >= 64 ? 1 : 64 / G;
    const uint64_t waves_needed = ((uint64_t)rows + (uint64_t)rpw * kRowdotU - 1) / ((uint64_t)rpw * kRowdotU);
    const uint64_t blocks_needed = (waves_needed + 3) / 4;
    const uint32_t cap = (uint32_t)std::max(1, cus) * 4;
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(blocks_needed, cap));
}

hipError_t launch_rowdot(int fmt, uint32_t blocks, const RowdotParams& p, hipStream_t stream) {
    const dim3 grid(blocks), block(256);
    if (fmt == FMT_Q4) hipLaunchKernelGGL((rowdot_kernel<FMT_Q4, kRowdotU>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((rowdot_kernel<FMT_F16, 4>), grid, block, 0, stream, p);
    return hipGetLastError();
}

bool lmhead_supported(uint32_t cols) {
    return cols == 128 || cols == 256 || cols == 512 || cols == 1024 || cols == 2048;
}

uint32_t lmhead_tiles(uint32_t rows) {
    return (rows + 15u) / 16u;
}

uint32_t lmhead_blocks(uint32_t rows, int cus) {
    const uint32_t tiles = lmhead_tiles(rows);
    const int bpc = std::max(1, std::min(8, env_int("QORA_LM_BPC", 2)));   // workgroups per CU
    const uint64_t cap = (uint64_t)std::max(1, cus) * (uint64_t)bpc;
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>((tiles + 3u) / 4u, cap));
}

void lmhead_tile_bytes(uint32_t rows, uint32_t cols, uint64_t* w_bytes, uint64_t* s_bytes) {
    const uint64_t units = (uint64_t)lmhead_tiles(rows) * (cols / 128u);
    *w_bytes = units * 1024u;
    *s_bytes = units * 128u;
}

hipError_t launch_lmhead_pack(const uint8_t* w, const uint16_t* scales, uint32_t rows, uint32_t cols, uint8_t* tw,
                              uint32_t* ts, hipStream_t stream) {
    if (rows == 0 || !lmhead_supported(cols)) return hipErrorInvalidValue;
    const uint32_t tiles = lmhead_tiles(rows);
    const uint64_t threads = (uint64_t)tiles * (cols / 128u) * 64u;
    hipLaunchKernelGGL(lmhead_q4m_pack_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, stream, w,
                       scales, rows, cols, tiles, tw, ts);
    return hipGetLastError();
}

hipError_t launch_lmhead(uint32_t blocks, const LmHeadParams& p, hipStream_t stream) {
    if (p.rows == 0 || p.tiles != lmhead_tiles(p.rows) || blocks == 0) return hipErrorInvalidValue;
    const bool fixed = p.xacc != nullptr;
    if (fixed ? !p.gamma : !p.x) return hipErrorInvalidValue;
    const dim3 grid(blocks), block(256);
#define QORA_LM_CASE(COLS_, NP_)                                                                           \
    case COLS_:                                                                                            \
        if (fixed) hipLaunchKernelGGL((lmhead_q4m_kernel<NP_, true>), grid, block, 0, stream, p);          \
        else hipLaunchKernelGGL((lmhead_q4m_kernel<NP_, false>), grid, block, 0, stream, p);               \
        break;
    switch (p.cols) {
        QORA_LM_CASE(128, 2)
        QORA_LM_CASE(256, 4)
        QORA_LM_CASE(512, 8)
        QORA_LM_CASE(1024, 16)
        QORA_LM_CASE(2048, 32)
        default: return hipErrorInvalidValue;
    }
#undef QORA_LM_CASE
    return hipGetLastError();
}

hipError_t launch_argmax_finish(const ArgmaxFinishParams& p, hipStream_t stream) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(256), 0, stream, p);
    return hipGetLastError();
}

void attn_geometry(uint32_t positions, uint32_t* chunk, uint32_t* s_max) {
    uint32_t c = (positions + kAttnMaxSplits - 1) / kAttnMaxSplits;
    c = std::max<uint32_t>(kAttnSub, (c + kAttnSub - 1) / kAttnSub * kAttnSub);
    *chunk = c;
    *s_max = std::max<uint32_t>(1, (positions + c - 1) / c);
}

hipError_t launch_attn(const AttnParams& p, hipStream_t stream) {
    const dim3 grid(p.s_max, p.KVH);
    const bool lng = p.nsg > 1;
    if (lng && p.kv_f16 && (p.hd == 128 || p.hd == 64) && p.groups <= (uint32_t)kAttnMaxGroups &&
        !tuning_env("QORA_HIP_ATTN_STAGED")) {
        const dim3 grid_t(p.KVH, p.s_max);
        if (p.hd == 128) hipLaunchKernelGGL((attn_decode_direct_kernel<128>), grid_t, dim3(512), 0, stream, p.pos, p);
        else hipLaunchKernelGGL((attn_decode_direct_kernel<64>), grid_t, dim3(512), 0, stream, p.pos, p);
        return hipGetLastError();
    }
    const dim3 block(lng ? 256 * kAttnLongNsg : 256);
    // attn_decode_kernel takes the arguments of its first loads ahead of the
    // parameter block (preloaded into scalar registers at wave launch), the
    // small ones packed: hd | groups << 10 | KVH << 20, H | half << 16 |
    // use_rope << 31, ss_n | norm_n << 8
    if (!lng && (p.hd > 0x3FFu || p.groups > 0x3FFu || p.KVH > 0xFFFu || p.H > 0xFFFFu || p.half > 0x7FFFu ||
                 p.ss_n > 0xFFu || p.norm_n >= (1u << 24)))
        return hipErrorInvalidValue;
    const uint32_t shape = p.hd | (p.groups << 10) | (p.KVH << 20);
    const uint32_t hh = p.H | (p.half << 16) | (p.use_rope ? 0x80000000u : 0u);
    const uint32_t snn = p.ss_n | (p.norm_n << 8);
#define QORA_ATTN(DPL)                                                                                   \
    do {                                                                                                \
        if (lng && p.kv_f16) hipLaunchKernelGGL((attn_decode_long_kernel<DPL, true>), grid, block, 0, stream, p); \
        else if (lng) hipLaunchKernelGGL((attn_decode_long_kernel<DPL, false>), grid, block, 0, stream, p); \
        else if (p.kv_f16)                                                                              \
            hipLaunchKernelGGL((attn_decode_kernel<DPL, true>), grid, block, 0, stream, p.pos, p.qkv_acc, p.ss_in, \
                               p.rope_cos, p.rope_sin, shape, hh, snn, p.chunk, p);                    \
        else                                                                                            \
            hipLaunchKernelGGL((attn_decode_kernel<DPL, false>), grid, block, 0, stream, p.pos, p.qkv_acc, p.ss_in, \
                               p.rope_cos, p.rope_sin, shape, hh, snn, p.chunk, p);                    \
    } while (0)
    if (p.hd <= 64) QORA_ATTN(1);
    else QORA_ATTN(2);
#undef QORA_ATTN
    return hipGetLastError();
}

bool attn_o_supported(const GemvPlan& pl, uint32_t hd, uint32_t H, uint32_t groups) {
    return pl.mfma && pl.gw == 1 && pl.ipw <= 1 && pl.kr == hd && pl.splits == H && (hd == 64 || hd == 128) &&
           groups >= 1 && groups <= (uint32_t)kAttnMaxGroups;
}

template <int HD, bool F16KV, bool CH>
static hipError_t launch_attn_o_hd(const GemvPlan& pl, const AttnOParams& p, uint32_t np, hipStream_t stream) {
    const dim3 grid(pl.blocks()), block(kFusedWaves * kWave);
    // the first loads' arguments go ahead of the parameter block (preloaded
    // into scalar registers at wave launch): the cache, the position, the
    // q|k|v sums and norm partials, tiles | groups << 16, KVH | half << 12 |
    // ss_n << 24 and the cache's position and head strides (in elements)
    const AttnParams& a = p.a;
    const uint64_t cps = a.kv_ps ? a.kv_ps : (uint64_t)a.KVH * a.hd, hs = a.kv_ps ? a.kv_hs : (uint64_t)a.hd;
    if (p.g.tiles > 0xFFFFu || a.groups > 0xFFFFu || a.KVH > 0xFFFu || a.half > 0xFFFu || a.ss_n > 0xFFu ||
        a.H != a.KVH * a.groups || pl.blocks() != p.g.tiles * a.H || cps > 0xFFFFFFFFull || hs > 0xFFFFFFFFull)
        return hipErrorInvalidValue;
    const uint32_t tg = p.g.tiles | (a.groups << 16), khs = a.KVH | (a.half << 12) | (a.ss_n << 24);
#define QORA_AO_ARGS p.a.kc, p.a.vc, p.a.pos, p.a.qkv_acc, p.a.ss_in, tg, khs, (uint32_t)cps, (uint32_t)hs, p
    switch (np) {
    case 1: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 1, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 2: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 2, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 3: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 3, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 4: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 4, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 5: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 5, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 6: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 6, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 7: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 7, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    case 8: hipLaunchKernelGGL((gemv_q4m_attn_kernel<HD, F16KV, 8, CH>), grid, block, 0, stream, QORA_AO_ARGS); break;
    default: return hipErrorInvalidValue;
    }
#undef QORA_AO_ARGS
    return hipGetLastError();
}

hipError_t launch_attn_o(const GemvPlan& pl, const AttnOParams& p, uint32_t np, bool chunked, hipStream_t stream) {
    if (chunked && !p.ch_count) return hipErrorInvalidValue;
    if (p.a.hd == 128) {
        if (chunked)
            return p.a.kv_f16 ? launch_attn_o_hd<128, true, true>(pl, p, np, stream)
                              : launch_attn_o_hd<128, false, true>(pl, p, np, stream);
        return p.a.kv_f16 ? launch_attn_o_hd<128, true, false>(pl, p, np, stream)
                          : launch_attn_o_hd<128, false, false>(pl, p, np, stream);
    }
    if (chunked)
        return p.a.kv_f16 ? launch_attn_o_hd<64, true, true>(pl, p, np, stream)
                          : launch_attn_o_hd<64, false, true>(pl, p, np, stream);
    return p.a.kv_f16 ? launch_attn_o_hd<64, true, false>(pl, p, np, stream)
                      : launch_attn_o_hd<64, false, false>(pl, p, np, stream);
}

bool attn_chunk_supported(const GemvPlan& pl, uint32_t hd, uint32_t H, uint32_t groups, uint32_t s_max, int cus) {
    if (!attn_o_supported(pl, hd, H, groups) || pl.tiles > kChunkMaxTiles || H > kChunkHeads || pl.tiles > s_max)
        return false;
    // every workgroup of a launch waits for the other column tiles of its
    // head: the grid must be resident at once
    int per_cu = 0;
    const hipError_t e =
        hd == 128 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_q4m_attn_kernel<128, false, 8, true>,
                                                                 kFusedWaves * kWave, 0)
                  : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_q4m_attn_kernel<64, false, 8, true>,
                                                                 kFusedWaves * kWave, 0);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return (uint64_t)pl.blocks() <= (uint64_t)per_cu * (uint64_t)std::max(cus, 1);
}

hipError_t launch_attn_combine(const AttnCombineParams& p, hipStream_t stream) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3(p.H), dim3(128), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_embed(const EmbedParams& p, hipStream_t stream) {
    const uint32_t blocks = std::max(1u, std::min(64u, (p.hidden + 255) / 256));
    hipLaunchKernelGGL(embed_kernel, dim3(blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_dequant_q4(const uint8_t* packed, const uint16_t* scales, uint64_t k, uint64_t n, float* out,
                             hipStream_t stream) {
    const uint64_t bytes = k * n / 2;
    const uint32_t blocks = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(4096, (bytes + 255) / 256));
    hipLaunchKernelGGL(dequant_q4_kernel, dim3(blocks), dim3(256), 0, stream, packed, scales, k, n, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const uint16_t* gamma, uint32_t n, float* out, hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, stream, x, gamma, n, out);
    return hipGetLastError();
}

hipError_t launch_rope(float* data, uint32_t heads, uint32_t head_dim, const float* cos_t, const float* sin_t,
                       uint32_t half, uint32_t position, hipStream_t stream) {
    const uint32_t total = heads * half;
    const uint32_t blocks = std::max(1u, std::min(256u, (total + 255) / 256));
    hipLaunchKernelGGL(rope_kernel, dim3(blocks), dim3(256), 0, stream, data, heads, head_dim, cos_t, sin_t, half,
                       position);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, uint32_t n, int32_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, stream, logits, n, out);
    return hipGetLastError();
}

hipError_t launch_advance_pos(int32_t* pos, hipStream_t stream) {
    hipLaunchKernelGGL(advance_pos_kernel, dim3(1), dim3(64), 0, stream, pos);
    return hipGetLastError();
}

// ---- batched prefill ----

// Register-cached row producers: rows of up to 4096 elements on 256 threads
// (8 or 16 per thread), SwiGLU rows of up to 12288 on 1024 threads (12 per
// thread); wider rows go to the two- or three-pass kernels.
template <int EPT>
static void launch_pf_rows_reg(int kind, const PrefillRowParams& p, uint32_t T, hipStream_t stream) {
    switch (kind) {
    case PF_ROW_RMSNORM: hipLaunchKernelGGL((pf_rmsnorm_split_reg_kernel<EPT>), dim3(T), dim3(256), 0, stream, p); break;
    case PF_ROW_SPLIT: hipLaunchKernelGGL((pf_split_reg_kernel<EPT>), dim3(T), dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL((pf_silu_split_reg_kernel<256, EPT>), dim3(T), dim3(256), 0, stream, p); break;
    }
}

static bool pf_rows_reg(int kind, const PrefillRowParams& p, uint32_t T, hipStream_t stream) {
    if (kind != PF_ROW_RMSNORM && kind != PF_ROW_SPLIT && kind != PF_ROW_SILU) return false;
    if (p.n <= 256u * 8u) launch_pf_rows_reg<8>(kind, p, T, stream);
    else if (p.n <= 256u * 16u) launch_pf_rows_reg<16>(kind, p, T, stream);
    else if (kind == PF_ROW_SILU && p.n <= 1024u * 12u)
        hipLaunchKernelGGL((pf_silu_split_reg_kernel<1024, 12>), dim3(T), dim3(1024), 0, stream, p);
    else return false;
    return true;
}

hipError_t launch_pf_rows(int kind, const PrefillRowParams& p, uint32_t T, hipStream_t stream) {
    if (T == 0) return hipSuccess;
    // QORA_HIP_PF_ROWS=loop keeps every row on the multi-pass kernels
    const char* er = tuning_env("QORA_HIP_PF_ROWS");
    const bool loop = er && std::strcmp(er, "loop") == 0;
    if (!loop && pf_rows_reg(kind, p, T, stream)) return hipGetLastError();
    switch (kind) {
    case PF_ROW_EMBED: hipLaunchKernelGGL(pf_embed_kernel, dim3(T), dim3(256), 0, stream, p); break;
    case PF_ROW_RMSNORM: hipLaunchKernelGGL(pf_rmsnorm_split_kernel, dim3(T), dim3(256), 0, stream, p); break;
    case PF_ROW_SPLIT: hipLaunchKernelGGL(pf_split_kernel, dim3(T), dim3(256), 0, stream, p); break;
    case PF_ROW_SILU: hipLaunchKernelGGL(pf_silu_split_kernel, dim3(T), dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

uint64_t pf_weight_exp_scratch(uint32_t k, uint32_t groups) {
    return (uint64_t)((k + kPfExpRows - 1) / kPfExpRows) * groups * 4;
}

hipError_t launch_pf_weight_exp(const uint16_t* scales, uint32_t k, uint32_t groups, int8_t* wf, uint32_t* scratch,
                                hipStream_t stream) {
    const uint32_t nblk = (k + kPfExpRows - 1) / kPfExpRows;
    hipLaunchKernelGGL(pf_weight_exp_part_kernel, dim3((groups + kWave - 1) / kWave, nblk), dim3(256), 0, stream,
                       scales, k, groups, scratch);
    hipLaunchKernelGGL(pf_weight_exp_kernel, dim3((groups + 255) / 256), dim3(256), 0, stream, scratch, nblk, groups,
                       wf);
    return hipGetLastError();
}

bool pf_gemm_supported(uint32_t k, uint32_t n) { return k > 0 && k % 32 == 0 && n >= 2 && n % 2 == 0; }

// Launch shape of the prefill GEMM: 128-column tiles when they still give
// every CU a block, else 64; then split K (into runs of at least 256 rows)
// until about four blocks per CU are in flight (four fit at once), since
// each block's K loop is bound by its global-load latency.
PfGemmShape pf_gemm_shape(uint32_t T, uint32_t k, uint32_t n, int cus) {
    PfGemmShape sh{};
    const uint32_t mt = (T + 63) / 64;
    const char* ev = tuning_env("QORA_HIP_PF_NT");
    bool wide = n % 128 == 0 && (uint64_t)(n / 128) * mt >= (uint64_t)cus;
    if (ev && *ev) wide = std::atoi(ev) == 128 && n % 128 == 0;
    sh.nt = wide ? 128 : 64;
    const uint64_t blocks = (uint64_t)((n + sh.nt - 1) / sh.nt) * mt;
    uint32_t splits = (uint32_t)std::min<uint64_t>(std::max<uint64_t>(1, (4ull * cus) / blocks), std::max(1u, k / 256));
    const char* es = tuning_env("QORA_HIP_PF_SPLITS");
    if (es && *es) splits = std::max(1, std::atoi(es));
    const uint32_t steps = k / 32;
    splits = std::min(splits, steps);
    const uint32_t per = (steps + splits - 1) / splits;
    sh.kper = per * 32;
    sh.splits = (steps + per - 1) / per;
    return sh;
}

hipError_t launch_pf_gemm(int fmt, const PrefillGemmParams& p, hipStream_t stream) {
    if (!pf_gemm_supported(p.k, p.n) || p.T == 0 || p.splits == 0 || p.kper % 32 != 0 ||
        (uint64_t)p.splits * p.kper < p.k || (p.splits > 1 && !p.part))
        return hipErrorInvalidValue;
    const uint32_t nt = (p.n % 128 == 0 && p.nt == 128) ? 128 : 64;
    const dim3 grid((p.n + nt - 1) / nt, (p.T + 63) / 64, p.splits);
    // QORA_HIP_PF_MODE=0 selects the double-buffered K loop (pf_gemm_kernel MODE 0)
    const char* em = tuning_env("QORA_HIP_PF_MODE");
    const int mode = (em && *em && std::atoi(em) == 0) ? 0 : 1;
#define QORA_PF_GEMM(NT_, Q4_)                                                                              \
    do {                                                                                                   \
        if (mode == 0) hipLaunchKernelGGL((pf_gemm_kernel<NT_, Q4_, 0>), grid, dim3(256), 0, stream, p);  \
        else hipLaunchKernelGGL((pf_gemm_kernel<NT_, Q4_, 1>), grid, dim3(256), 0, stream, p);            \
    } while (0)
    if (fmt == FMT_Q4) {
        if (nt == 128) QORA_PF_GEMM(128, true);
        else QORA_PF_GEMM(64, true);
    } else {
        if (nt == 128) QORA_PF_GEMM(128, false);
        else QORA_PF_GEMM(64, false);
    }
#undef QORA_PF_GEMM
    if (p.splits > 1) {
        const uint64_t total = (uint64_t)p.T * p.n;
        const uint32_t blocks = (uint32_t)std::min<uint64_t>(4096, (total + 255) / 256);
        hipLaunchKernelGGL(pf_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

bool pf_gemm2_supported(uint32_t k, uint32_t n) { return k > 0 && k % 32 == 0 && n > 0 && n % 128 == 0; }

hipError_t launch_pf_pack_q4(const uint8_t* w, const uint16_t* scales, const int8_t* wf, uint32_t k, uint32_t n,
                             uint2* wq, uint16_t* sc, hipStream_t stream) {
    if (!pf_gemm2_supported(k, n) || !wf) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_pack_q4_kernel, dim3(n / 128, k / 32), dim3(256), 0, stream, w, scales, wf, k, n, wq, sc);
    return hipGetLastError();
}

// Tile height (32 or 64 tokens), then the K split.
PfGemm2Shape pf_gemm2_shape(uint32_t T, uint32_t k, uint32_t ntot, int cus) {
    PfGemm2Shape sh{};
    const uint32_t steps = k / 32u;
    const uint64_t cu = (uint64_t)std::max(1, cus);
    // 64-token tiles; 32-token tiles where K is short (at most 4096) and the
    // 64-token tiles leave two block slots per CU partly empty: twice the
    // blocks without more split partials (512 tokens on 256 CUs: q|k|v and o;
    // a long K such as down's 11008 streams twice the weights through the L2
    // with 32-token tiles and measured slower)
    sh.bm = 64u;
    if (k <= 4096u && (uint64_t)(ntot / 128u) * ((T + 63u) / 64u) < 2u * cu) sh.bm = 32u;
    const char* eb = tuning_env("QORA_HIP_PF_BM");
    if (eb && *eb) sh.bm = std::atoi(eb) == 32 ? 32u : 64u;     // tuning and tests: force 32 or 64
    const uint64_t tiles = std::max<uint64_t>(1, (uint64_t)(ntot / 128u) * ((T + sh.bm - 1) / sh.bm));
    // K is split only when the tiles leave the block slots partly empty (two
    // per CU; three for the lighter 32-token blocks): beyond that a split's
    // partial-sum traffic costs more than it gains. The splits are of equal
    // length (at least 8 steps each, at most 16 splits), and the count is the
    // one whose blocks fill their rounds best (fewer splits unless more fill
    // them better by 2% or more): 512 tokens on 256 CUs, q|k|v 2 and o 3 with
    // 32-token tiles, gate|up 1 and down 4 with 64-token tiles.
    const uint64_t slots = (sh.bm == 32u ? 3u : 2u) * cu;
    const uint32_t smax = tiles >= slots ? 1u
                                         : (uint32_t)std::min<uint64_t>({16u, std::max(1u, steps / 8u),
                                                                         (slots + tiles - 1) / tiles});
    uint32_t splits = 1;
    double best = -1.0;
    for (uint32_t s = 1; s <= smax; ++s) {
        const uint32_t per = (steps + s - 1) / s;
        if ((steps + per - 1) / per != s) continue;
        const uint64_t blocks = tiles * s, rounds = (blocks + slots - 1) / slots;
        const double fill = (double)blocks / (double)(rounds * slots);
        if (fill > best + 0.02) {
            best = fill;
            splits = s;
        }
    }
    const char* es = tuning_env("QORA_HIP_PF_SPLITS");
    if (es && *es) splits = std::min(std::max(1, std::atoi(es)), (int)std::max(1u, steps / 8u));
    const uint32_t per = (steps + splits - 1) / splits;
    sh.kper = per * 32u;
    sh.splits = (steps + per - 1) / per;
    return sh;
}

hipError_t launch_pf_gemm2(uint32_t bm, const PfGemm2Params& p, hipStream_t stream, bool reduce) {
    if (p.T == 0 || p.k % 32 != 0 || p.nseg < 1 || p.nseg > 3 || p.ntot % 128 != 0 || p.splits == 0 ||
        p.kper % 32 != 0 || (uint64_t)p.splits * p.kper < p.k || (p.splits > 1 && !p.part))
        return hipErrorInvalidValue;
    uint32_t nb = 0;
    for (int i = 0; i < p.nseg; ++i) {
        if (p.seg[i].nb0 != nb || p.seg[i].n % 128 != 0 || !p.seg[i].wq || !p.seg[i].sc || !p.seg[i].wf) return hipErrorInvalidValue;
        nb += p.seg[i].n / 128;
    }
    if (nb * 128u != p.ntot) return hipErrorInvalidValue;
    if (p.swiglu && (p.nseg != 2 || p.seg[0].n != p.seg[1].n || p.splits != 1 || !p.seg[0].y || p.seg[0].accumulate))
        return hipErrorInvalidValue;
    const dim3 grid(nb, (p.T + bm - 1) / bm, p.splits);
    if (bm == 64) hipLaunchKernelGGL((pf_gemm2_kernel<64>), grid, dim3(256), 0, stream, p);
    else if (bm == 32) hipLaunchKernelGGL((pf_gemm2_kernel<32>), grid, dim3(256), 0, stream, p);
    else return hipErrorInvalidValue;
    if (p.splits > 1 && reduce) {
        const uint64_t total = (uint64_t)p.T * p.ntot;
        const uint32_t blocks = (uint32_t)std::min<uint64_t>(4096, (total + 255) / 256);
        hipLaunchKernelGGL(pf_splitk_reduce2_kernel, dim3(blocks), dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

hipError_t launch_pf_rope_cache(const PrefillAttnParams& p, hipStream_t stream) {
    if (p.T == 0) return hipSuccess;
    if (p.kv_f16) hipLaunchKernelGGL((pf_rope_cache_kernel<true>), dim3(p.T), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((pf_rope_cache_kernel<false>), dim3(p.T), dim3(256), 0, stream, p);
    return hipGetLastError();
}

// The attention output rows (p.out) split into the o GEMM's operand.
static hipError_t launch_pf_attn_split(const PrefillAttnParams& p, hipStream_t stream) {
    PrefillRowParams r{};
    r.x = p.out;
    r.n = p.H * p.hd;
    r.xh = p.xh;
    r.xl = p.xl;
    r.xe = p.xe;
    return launch_pf_rows(PF_ROW_SPLIT, r, p.T, stream);
}

hipError_t launch_pf_attn(const PrefillAttnParams& p, hipStream_t stream) {
    if (p.T == 0) return hipSuccess;
    if (p.hd > (uint32_t)kAttnMaxHd || p.hd % 8 != 0 || p.H % p.KVH != 0) return hipErrorInvalidValue;
    const uint32_t G = p.H / p.KVH;
    if ((p.hd == 64 || p.hd == 128) && (G == 1 || G == 2 || G == 4)) {
        const uint32_t qt = 16u * (4u / G);
        // Key chunks: a query block's keys split over up to part_nc blocks
        // (128 keys each, more when that would exceed part_nc) so that the
        // long rows of the causal triangle do not set the kernel's length;
        // pf_attn_merge_kernel combines the chunks. QORA_HIP_PF_ATTN_CH sets
        // the chunk (a multiple of 64).
        PrefillAttnParams q = p;
        q.nc = 1;
        q.ch = 0;
        if (p.part && p.part_nc >= 2 && p.part_nc <= 8) {   // 8: pf_attn_merge_kernel's bound
            const uint32_t keys = p.pos0 + p.T;
            uint32_t ch = 128;
            const char* ec = tuning_env("QORA_HIP_PF_ATTN_CH");
            if (ec && *ec) ch = std::max(64u, (uint32_t)std::atoi(ec) / 64u * 64u);
            if ((keys + ch - 1) / ch > p.part_nc) ch = ((keys + p.part_nc - 1) / p.part_nc + 63u) / 64u * 64u;
            const uint32_t nc = (keys + ch - 1) / ch;
            if (nc >= 2) {
                q.nc = nc;
                q.ch = ch;
            }
        }
        const dim3 grid((p.T + qt - 1) / qt * q.nc, p.KVH);
        // with split outputs and chunks, the merge writes the o GEMM's operand itself
        const bool merge_split = p.xh && q.nc > 1 && p.H * p.hd <= 2048u;
#define QORA_PF_ATTN(HD)                                                                                     \
    do {                                                                                                    \
        if (p.kv_f16) hipLaunchKernelGGL((pf_attn_mfma_kernel<HD, true>), grid, dim3(256), 0, stream, q);   \
        else hipLaunchKernelGGL((pf_attn_mfma_kernel<HD, false>), grid, dim3(256), 0, stream, q);           \
        if (merge_split)                                                                                    \
            hipLaunchKernelGGL((pf_attn_merge_split_kernel<HD>), dim3(p.T), dim3(256), 0, stream, q);        \
        else if (q.nc > 1)                                                                                  \
            hipLaunchKernelGGL((pf_attn_merge_kernel<HD>), dim3(p.T, (p.H * HD + 255) / 256), dim3(256), 0,  \
                               stream, q);                                                                  \
    } while (0)
        if (p.hd == 128) QORA_PF_ATTN(128);
        else QORA_PF_ATTN(64);
#undef QORA_PF_ATTN
        if (p.xh && !merge_split) return launch_pf_attn_split(p, stream);
        return hipGetLastError();
    }
    const dim3 grid((p.T + 31) / 32, p.H);
    if (p.kv_f16) hipLaunchKernelGGL((pf_attn_vec_kernel<true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((pf_attn_vec_kernel<false>), grid, dim3(256), 0, stream, p);
    if (p.xh) return launch_pf_attn_split(p, stream);
    return hipGetLastError();
}

// ---- on-device sampling ----

uint32_t smp_blocks(uint32_t vocab) { return (vocab + kSmpBlock - 1) / kSmpBlock; }
bool smp_supported(uint32_t vocab) { return vocab > 0 && smp_blocks(vocab) * kSmpKeep <= kSmpFinal; }

hipError_t launch_sample(const float* logits, const SampleParams& p, hipStream_t stream) {
    if (!smp_supported(p.vocab) || p.blocks != smp_blocks(p.vocab) || p.top_k == 0 || p.top_k > kSmpKeep)
        return hipErrorInvalidValue;
    // the block kernel reads the logits and applies the penalties itself
    SampleParams q = p;
    q.logits = logits;
    hipLaunchKernelGGL(smp_block_topk_kernel, dim3(p.blocks), dim3(kSmpTopkThreads), 0, stream, q);
    hipLaunchKernelGGL(smp_final_kernel, dim3(1), dim3(kSmpFinalThreads), 0, stream, q);
    return hipGetLastError();
}

uint32_t smp_sort_keys(uint32_t vocab) {
    uint32_t n = smp_blocks(vocab) * kSmpBlock, m = kSmpBlock;
    while (m < n) m <<= 1;
    return m;
}
bool smp_sort_supported(uint32_t vocab) { return vocab > 0 && vocab <= kSmpSortMax; }

hipError_t launch_sample_sorted(const float* logits, const SampleParams& p, uint32_t k, hipStream_t stream) {
    if (!smp_sort_supported(p.vocab) || p.blocks != smp_blocks(p.vocab) || p.n_sort != smp_sort_keys(p.vocab) ||
        k == 0 || k > p.vocab || !p.sort_a || !p.sort_b || !p.probs)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(smp_copy_kernel, dim3(std::min<uint32_t>(1024, (p.vocab + 255) / 256)), dim3(256), 0, stream,
                       logits, p.work, p.vocab);
    if (p.n_pen) hipLaunchKernelGGL(smp_penalty_kernel, dim3((p.n_pen + 255) / 256), dim3(256), 0, stream, p);
    // runs of 2048 keys (the padding blocks past the vocabulary sort to all ~0)
    const uint32_t nb = p.n_sort / kSmpBlock;
    SampleParams q = p;
    hipLaunchKernelGGL(smp_block_sort_kernel, dim3(nb), dim3(256), 0, stream, q);
    unsigned long long* src = p.sort_a;
    unsigned long long* dst = p.sort_b;
    for (uint32_t run = kSmpBlock; run < p.n_sort; run <<= 1) {
        hipLaunchKernelGGL(smp_merge_kernel, dim3(p.n_sort / 256), dim3(256), 0, stream, (const unsigned long long*)src,
                           dst, p.n_sort, run);
        std::swap(src, dst);
    }
    if (p.temperature > 0.0f)
        hipLaunchKernelGGL(smp_probs_kernel, dim3((k + 255) / 256), dim3(256), 0, stream, p,
                           (const unsigned long long*)src, k);
    hipLaunchKernelGGL(smp_scan_kernel, dim3(1), dim3(256), 0, stream, p, (const unsigned long long*)src, k);
    return hipGetLastError();
}

}  // namespace qora
