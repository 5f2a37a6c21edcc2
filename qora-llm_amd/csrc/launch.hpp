// Host-side launch helpers for the decode kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "params.hpp"

namespace qora {

// Value of a tuning or test variable (launch-shape overrides, test hooks):
// read only when QORA_HIP_TUNING=1 is set, so a host that inherits such a
// variable does not change the kernels by accident; nullptr otherwise.
const char* tuning_env(const char* name);

// Launch shape of one split-K GEMV call site.
struct GemvPlan {
    int gt = 8;           // groups per column tile
    int rpl = 4;          // rows per lane (VALU kernel)
    uint32_t tiles = 0;   // column tiles
    uint32_t splits = 0;  // K slices
    uint32_t kr = 0;      // rows per K slice
    int mfma = 0;         // 1: Q4 on the matrix cores (gemv_q4m_kernel): gt = 4*gw, kr = kw
    int gw = 0;           // groups per wave (MFMA kernel)
    int ipw = 1;          // work items (tile, K slice) per workgroup (MFMA kernel)
    uint32_t blocks() const { return tiles * splits; }                // work items
    uint32_t grid() const { return (blocks() + (uint32_t)ipw - 1) / (uint32_t)ipw; }
};

// Chooses GT / RPL / S for k input rows. seg_groups: groups (n/32) of each
// segment; paired: gate/up lane pairing (two segments of equal groups).
// cus: compute units on the device. Returns false if the shape is unsupported.
// row_align (optional): K slices must start on multiples of it (head_dim
// for the attention-merge prologue).
bool plan_gemv(int fmt, uint32_t k, const uint32_t* seg_groups, int nseg, bool paired, int cus, GemvPlan* plan,
               uint32_t row_align = 1);

// Q4 GEMV on the matrix cores: one group per wave (QORA_GEMV_GW may force 2
// or 4) and the deepest K slice of 256, 128 or 64 rows (QORA_GEMV_KW may
// force one) that gives every CU a workgroup.
// force_kw (256, 128 or 64): that K slice and one group per wave, whatever the
// environment says.
bool plan_gemv_q4m(uint32_t k, const uint32_t* seg_groups, int nseg, bool paired, int cus, GemvPlan* plan,
                   uint32_t row_align = 1, uint32_t force_kw = 0);

// Fills seg[].tile0/tiles/col0 and p.tiles/splits/rows_per_split from the plan.
// Concatenated segments land one after the other in the accumulator; paired
// segments at 0 (gate) and n (up).
void apply_plan(const GemvPlan& plan, GemvParams* p);

// p.tw == nullptr: reference layout, plain prologue only (kernel-level
// entry points). Otherwise the tile layout written by launch_gemv_tile.
hipError_t launch_gemv(int fmt, const GemvPlan& plan, const GemvParams& p, hipStream_t stream);
// Size of the tile layout of a planned GEMV (scales, exponent bounds: Q4 only).
void gemv_tile_bytes(int fmt, const GemvPlan& plan, uint64_t* w_bytes, uint64_t* s_bytes, uint64_t* e_bytes);
// Writes the tile layout of the reference-layout segments of p (after
// apply_plan) into tw / ts / te, sized by gemv_tile_bytes.
hipError_t launch_gemv_tile(int fmt, const GemvPlan& plan, const GemvParams& p, uint8_t* tw, uint16_t* ts,
                            int8_t* te, hipStream_t stream);
hipError_t launch_fill_zero(long long* p, uint64_t n, hipStream_t stream);
// One layer's KV cache [kvh][cap][hd] (f32, or binary16 rounded to nearest even) from / to the
// token-major rows [len][kvh][hd] f32 (to_cache: rows -> cache).
hipError_t launch_kv_move(bool to_cache, bool f16, float* rows, void* cache, uint32_t len, uint32_t kvh, uint32_t hd,
                          uint64_t cap, hipStream_t stream);
hipError_t launch_acc_to_f32(const long long* acc, uint32_t n, int paired, float* y, hipStream_t stream);

// Row-dot GEMV (lm_head). blocks: grid size (also the argmax partial count).
uint32_t rowdot_blocks(uint32_t rows, uint32_t cols, int cus);
hipError_t launch_rowdot(int fmt, uint32_t blocks, const RowdotParams& p, hipStream_t stream);
hipError_t launch_argmax_finish(const ArgmaxFinishParams& p, hipStream_t stream);

// Tied lm_head on the matrix cores (Q4, cols in {128, 256, 512, 1024, 2048}).
// blocks: grid size (also the argmax partial count).
bool lmhead_supported(uint32_t cols);
uint32_t lmhead_tiles(uint32_t rows);
uint32_t lmhead_blocks(uint32_t rows, int cus);
void lmhead_tile_bytes(uint32_t rows, uint32_t cols, uint64_t* w_bytes, uint64_t* s_bytes);
hipError_t launch_lmhead_pack(const uint8_t* w, const uint16_t* scales, uint32_t rows, uint32_t cols, uint8_t* tw,
                              uint32_t* ts, hipStream_t stream);
hipError_t launch_lmhead(uint32_t blocks, const LmHeadParams& p, hipStream_t stream);

// Attention split geometry for up to `positions` positions: chunk is a
// multiple of kAttnSub and s_max = ceil(positions / chunk) <= kAttnMaxSplits.
void attn_geometry(uint32_t positions, uint32_t* chunk, uint32_t* s_max);
hipError_t launch_attn(const AttnParams& p, hipStream_t stream);
hipError_t launch_attn_combine(const AttnCombineParams& p, hipStream_t stream);
// Short-context decode: attention of each query head in the o GEMV's
// prologue (gemv_q4m_attn_kernel). The o plan must be an MFMA plan with one
// group per wave and K slices of exactly one head (kr = hd, splits = H).
bool attn_o_supported(const GemvPlan& pl, uint32_t hd, uint32_t H, uint32_t groups);
// The fused short-context step for contexts of 32 (np - 1) < L <= 32 np positions, np in 1..8;
// chunked: the chunked step, each column tile over 32 np positions (tiles * 32 np >= L).
hipError_t launch_attn_o(const GemvPlan& pl, const AttnOParams& p, uint32_t np, bool chunked, hipStream_t stream);
// The chunked step on this plan: at most kChunkMaxTiles column tiles, a.part
// large enough for H * tiles states (tiles <= s_max), the grid resident at once.
bool attn_chunk_supported(const GemvPlan& pl, uint32_t hd, uint32_t H, uint32_t groups, uint32_t s_max, int cus);

hipError_t launch_embed(const EmbedParams& p, hipStream_t stream);
hipError_t launch_dequant_q4(const uint8_t* packed, const uint16_t* scales, uint64_t k, uint64_t n,
                             float* out, hipStream_t stream);
hipError_t launch_rmsnorm(const float* x, const uint16_t* gamma, uint32_t n, float* out, hipStream_t stream);
hipError_t launch_rope(float* data, uint32_t heads, uint32_t head_dim, const float* cos_t, const float* sin_t,
                       uint32_t half, uint32_t position, hipStream_t stream);
hipError_t launch_argmax(const float* logits, uint32_t n, int32_t* out, hipStream_t stream);
hipError_t launch_advance_pos(int32_t* pos, hipStream_t stream);

// batched prefill (prefill.hpp)
enum PfRow : int { PF_ROW_EMBED = 0, PF_ROW_RMSNORM = 1, PF_ROW_SPLIT = 2, PF_ROW_SILU = 3 };
hipError_t launch_pf_rows(int kind, const PrefillRowParams& p, uint32_t T, hipStream_t stream);
// per-group weight exponents; scratch holds pf_weight_exp_scratch(k, groups) bytes
uint64_t pf_weight_exp_scratch(uint32_t k, uint32_t groups);
hipError_t launch_pf_weight_exp(const uint16_t* scales, uint32_t k, uint32_t groups, int8_t* wf, uint32_t* scratch,
                                hipStream_t stream);
bool pf_gemm_supported(uint32_t k, uint32_t n);
struct PfGemmShape {
    uint32_t nt, splits, kper;
};
PfGemmShape pf_gemm_shape(uint32_t T, uint32_t k, uint32_t n, int cus);
// p.nt, p.splits, p.kper from pf_gemm_shape; p.part holds splits * T * n floats when splits > 1
hipError_t launch_pf_gemm(int fmt, const PrefillGemmParams& p, hipStream_t stream);
// Prefill GEMM on pre-packed Q4 weights (pf_gemm2_kernel). pack: the packed
// copy of a Q4 weight [k][n] (k % 32 == 0, n % 128 == 0) into wq (k n / 2
// bytes) and sc (k n / 16 bytes, the scales times 2^-wf[group]); wf from
// launch_pf_weight_exp.
bool pf_gemm2_supported(uint32_t k, uint32_t n);
hipError_t launch_pf_pack_q4(const uint8_t* w, const uint16_t* scales, const int8_t* wf, uint32_t k, uint32_t n,
                             uint2* wq, uint16_t* sc, hipStream_t stream);
struct PfGemm2Shape {
    uint32_t bm, splits, kper;
};
PfGemm2Shape pf_gemm2_shape(uint32_t T, uint32_t k, uint32_t ntot, int cus);
// p.splits, p.kper from pf_gemm2_shape (bm too); p.part holds splits * T * ntot floats when splits > 1.
// reduce = false leaves the split partials for the consumer to sum (pf_rmsnorm_split_reg_kernel).
hipError_t launch_pf_gemm2(uint32_t bm, const PfGemm2Params& p, hipStream_t stream, bool reduce = true);
hipError_t launch_pf_rope_cache(const PrefillAttnParams& p, hipStream_t stream);
hipError_t launch_pf_attn(const PrefillAttnParams& p, hipStream_t stream);

// on-device sampling (sample.hpp): vocab <= 131072, 1 <= top_k <= 64
uint32_t smp_blocks(uint32_t vocab);
bool smp_supported(uint32_t vocab);
hipError_t launch_sample(const float* logits, const SampleParams& p, hipStream_t stream);
// The full-sort path (any top_k, vocabularies up to 4M): n_sort keys per
// sort buffer, and the kernels over the first k sorted candidates.
uint32_t smp_sort_keys(uint32_t vocab);
bool smp_sort_supported(uint32_t vocab);
hipError_t launch_sample_sorted(const float* logits, const SampleParams& p, uint32_t k, hipStream_t stream);

}  // namespace qora
