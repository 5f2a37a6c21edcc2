// Launch-parameter structs shared by the kernels and the host launch code.
#pragma once

#include <stdint.h>

namespace qora {

enum WFmt : int { FMT_F16 = 0, FMT_Q4 = 1 };

// Where a GEMV workgroup gets the input rows of its K slice.
enum Pro : int {
    PRO_PLAIN = 0,        // fp32 vector x[k]
    PRO_GAMMA_FIXED = 1,  // x * gamma, x = the fixed-point residual xacc[k]. The RMSNorm
                          // factor is a scalar, so it is applied by the consumer of the
                          // output; workgroups of column tile 0 write sum(x^2) of their
                          // K slice to ss_out[split] for it.
    PRO_SILU_FIXED = 2,   // silu(inv * g) * (inv * u), g = xacc[0:k], u = xacc[k:2k], with
                          // inv = RMSNorm factor from the ss_in partials
    PRO_ATTN = 3,         // merge of the split attention partials of the heads in the slice
};

// Fixed-point accumulators: value = int64 / 2^36. Integer adds are exact and
// associative, so the split-K sums are identical whatever order the
// workgroups finish in. Resolution 1.5e-11. Range guard: a value read from
// the residual must be below 2^25 in magnitude (|int| < 2^61) and a single
// added contribution below 2^20 (|int| < 2^56); an accumulator takes at most
// kFixMaxTerms contributions between two reads (the launch planners enforce
// it), so a value in range when read cannot wrap before the next read:
// |int| < 2^61 + 96 * 2^56 = 2^63. Kernels given a range_flag set it when a
// value breaks either bound; the host reports QORA_HIP_E_RANGE.
constexpr double kFixScale = 68719476736.0;   // 2^36
constexpr long long kFixReadLimit = 1LL << 61;
constexpr long long kFixAddLimit = 1LL << 56;
constexpr uint32_t kFixMaxTerms = 96;

struct GemvSeg {
    const uint8_t* w;         // Q4 packed bytes or F16 words (as bytes), reference layout
    const uint16_t* scales;   // Q4 only
    uint32_t groups;          // n / 32
    uint32_t tile0;           // first column tile (concatenated mode)
    uint32_t tiles;           // column tiles of this segment
    uint32_t col0;            // output offset of this segment in the accumulator
};

struct GemvParams {
    GemvSeg seg[3];
    int nseg;
    int paired;               // 1: seg0 = gate, seg1 = up, lanes split in halves
    uint32_t k;
    uint32_t tiles;           // total column tiles
    uint32_t splits;          // S
    uint32_t rows_per_split;  // KR
    int pro;
    const float* x;           // PRO_PLAIN
    const long long* xacc;    // PRO_GAMMA_FIXED / PRO_SILU_FIXED input accumulator
    const uint16_t* gamma;    // PRO_GAMMA_FIXED
    float* ss_out;            // PRO_GAMMA_FIXED: sum of squares per K slice [splits]
    const float* ss_in;       // PRO_SILU_FIXED: partial sums of squares of the norm input
    uint32_t ss_n;            // number of ss_in partials (<= 64)
    uint32_t norm_n;          // length of the normalised vector
    // PRO_ATTN: attention partials [KVH][s_max][groups][head_dim + 2]
    const float* attn_part;
    uint32_t attn_s_max, attn_chunk, head_dim, groups;   // attn_chunk 0: attn_chunk_for(L)
    const int32_t* pos;
    long long* acc;           // output: fixed-point accumulator (+= W x)
    long long* zero_ptr;      // optional int64 buffer cleared by this launch
    uint32_t zero_n;
    // Tile layout (set by gemv_tile_kernel): the bytes every workgroup loads,
    // stored in load order so each workgroup streams one contiguous block.
    //   Q4 : tw[block][j < RPL][lane < 256] x 16 B, ts[block][lane][j] scales
    //   F16: tw[block][j][v < 4][lane] x 16 B
    // The segment pointers then only describe the shape.
    const uint8_t* tw;
    const uint16_t* ts;
    // Q4 on the matrix cores (gemv_q4m_kernel): per (workgroup, wave, group)
    // exponent bound of the K slice's scales, max |s| <= 2^tes.
    const int8_t* tes;
    int* range_flag;          // optional: set when a fixed-point value leaves its range
    // 1: the matrix-core kernels run item xcd_item(b, G) in workgroup b
    // (each XCD takes a contiguous run of items); 0: item b
    uint32_t xcd_order;
};

struct RowdotParams {
    const uint8_t* w;
    const uint16_t* scales;
    uint32_t rows, cols;       // cols = hidden, multiple of 32, cols/32 divides 64
    const float* x;            // fp32 input, or
    const long long* xacc;     // fixed-point residual (used when non-null)
    const uint16_t* gamma;     // optional RMSNorm prologue
    float* y;                  // [rows]
    int do_argmax;
    float* part_val;           // [gridDim.x] per-workgroup best logit
    uint32_t* part_idx;
    int* range_flag;           // optional: set when an xacc value leaves its range
};

// Row-dot Q4 GEMV on the matrix cores (lmhead_q4m_kernel): the tied lm_head,
// y[r] = sum_c x[c] * W[r][c] over W [rows][cols], groups of 32 along cols.
// Tile layout (lmhead_q4m_pack_kernel): 16 rows per tile, cols / 128
// 16-byte units per lane:
//   tw: [tile][unit][lane < 64] x 16 B   B fragments of column pairs 2u, 2u+1
//   ts: [tile][unit][lane < 32] x 4 B    two f16 scales of the lane's groups
struct LmHeadParams {
    const uint8_t* tw;
    const uint32_t* ts;
    uint32_t rows, cols;       // cols = 64 * NP
    uint32_t tiles;            // ceil(rows / 16)
    const float* x;            // fp32 input (used as is), or
    const long long* xacc;     // fixed-point residual with the RMSNorm prologue (when non-null)
    const uint16_t* gamma;     // RMSNorm gamma, required with xacc
    float* y;                  // [rows]
    int do_argmax;
    float* part_val;           // [gridDim.x] per-workgroup best logit
    uint32_t* part_idx;
    int* range_flag;           // optional: set when an xacc value leaves its range
};


// Batched prefill (prefill.hpp). Split GEMM operands: xh, xl binary16 words
// [T][k] and xe[T] exponents (x = (xh + xl) * 2^xe).
struct PrefillRowParams {
    const uint32_t* ids;       // pf_embed_kernel: token ids [T]
    uint32_t vocab;
    int fmt;
    const uint8_t* emb_w;
    const uint16_t* emb_s;
    float* x;                  // fp32 rows [T][ld] (embedding output, norm input, gate rows)
    const float* u;            // pf_silu_split_kernel: up rows [T][ld]
    uint32_t ld;               // row stride of x / u (pf_silu_split_kernel)
    uint32_t n;                // row length
    const uint16_t* gamma;     // pf_rmsnorm_split_kernel
    uint16_t* xh;
    uint16_t* xl;
    int32_t* xe;
    // pf_rmsnorm_split_reg_kernel: optional split-K partials of the GEMM that
    // produced x's increment, part[z][T][n] (z < splits, z-stride part_stride):
    // x += sum over z in split order (stored back), then the norm
    const float* part;
    uint32_t splits;
    uint64_t part_stride;
};

struct PrefillGemmParams {
    const uint16_t* xh;
    const uint16_t* xl;
    const int32_t* xe;
    uint32_t T, k, n;
    const uint8_t* w;          // reference layout: Q4 packed [k][n/2] or f16 [k][n]
    const uint16_t* scales;    // Q4 [k][n/32]
    const int8_t* wf;          // Q4 per-group exponents [n/32]
    float* y;                  // [T][ldy]
    uint32_t ldy;
    int accumulate;            // 1: y += result (residual add)
    // split K: grid.z = splits, split z takes rows [z kper, (z + 1) kper) and
    // writes its partial to part[z][T][n]; pf_splitk_reduce_kernel sums the
    // partials in split order into y
    uint32_t splits, kper;
    float* part;
    uint32_t nt;               // column tile (64 or 128), from pf_gemm_shape
};

// Pre-packed Q4 weight of the prefill GEMM (pf_gemm2_kernel): column block
// nb (128 columns), K step ks (32 rows), thread t = 64 rg + bc of a 256-thread
// block: wq[(nb * KS + ks) * 256 + t] holds 8 bytes, byte r = the two
// nibbles of columns 2 bc, 2 bc + 1 of row 32 ks + 8 rg + r (the reference
// byte); sc[((nb * KS + ks) * 4 + g) * 32 + r] the f16 scale of row 32 ks + r,
// group g of the block. KS = k / 32.
struct PfGemm2Seg {
    const uint2* wq;
    const uint16_t* sc;
    const int8_t* wf;          // per-group exponents [n/32]
    uint32_t n;                // columns (multiple of 128)
    uint32_t nb0;              // first column block of the segment in the grid
    float* y;                  // [T][ldy]
    uint32_t ldy;
    int accumulate;            // 1: y += result (residual add)
};

struct PfGemm2Params {
    const uint16_t* xh;
    const uint16_t* xl;
    const int32_t* xe;
    uint32_t T, k;
    PfGemm2Seg seg[3];
    int nseg;
    uint32_t ntot;             // columns of all segments
    // split K: grid.z = splits, split z takes rows [z kper, (z + 1) kper) and
    // writes part[z][T][ntot]; pf_splitk_reduce2_kernel sums them in split order
    uint32_t splits, kper;
    float* part;
    // SwiGLU pairing (gate|up): seg[0] = gate, seg[1] = up, both n wide, K
    // unsplit; column block b computes gate and up columns [64 b, 64 b + 64)
    // and writes h = SiLU(gate) * up to seg[0].y (row stride seg[0].ldy)
    int swiglu;
};

struct PrefillAttnParams {
    const float* qkv;          // GEMM output rows [T][qd + 2 kvd]
    float* q;                  // rotated q [T][qd]
    void* kc;                  // this layer's cache [cap][kvd]
    void* vc;
    int kv_f16;
    const float* rope_cos;
    const float* rope_sin;
    int use_rope;
    uint32_t half;
    uint32_t pos0;             // absolute position of the chunk's first token
    uint32_t T;                // tokens in the chunk
    uint32_t H, KVH, hd;
    float scale;
    float* out;                // attention output [T][qd]
    uint64_t kv_ps, kv_hs;     // cache addressing as in AttnParams (0: token-major)
    // key-range split of the matrix-core kernel: a workspace for up to part_nc
    // key chunks per query block (null / < 2: no split); nc and ch (keys per
    // chunk, a multiple of 64) are set by the launcher
    float* part;
    uint32_t part_nc;
    uint32_t nc, ch;
    // pf_rope_cache_kernel: optional split-K partials of the q|k|v GEMM,
    // qkv_part[z][T][qd + 2 kvd] (z-stride qkv_part_stride), summed in split
    // order in place of the qkv rows (rows of at most kPfRopeRowMax floats)
    const float* qkv_part;
    uint32_t qkv_splits;
    uint64_t qkv_part_stride;
    // optional: the attention output written as the o GEMM's operand (two
    // binary16 parts and a row exponent, as pf_split_kernel makes them)
    // instead of the fp32 rows in out
    uint16_t* xh;
    uint16_t* xl;
    int32_t* xe;
};
constexpr uint32_t kPfRopeRowMax = 8192;

// On-device sampling (sample.hpp).
struct SamplePenalty {
    uint32_t token;
    uint32_t rep_count;        // occurrences in the last 64 history tokens (repetition penalty)
    uint32_t seen;             // 1: the presence penalty applies
    uint32_t pad_;
};

struct SampleParams {
    float* work;               // [vocab] penalised copy of the logits
    uint32_t vocab;
    const SamplePenalty* pen;  // distinct history tokens
    uint32_t n_pen;
    float repetition, presence;
    unsigned long long* cand;  // [blocks][kSmpKeep] per-block best keys
    uint32_t blocks;
    float temperature, top_p;
    uint32_t top_k;
    unsigned long long rng_in; // xorshift64 state before the draw
    unsigned long long* rng;   // the state after it
    int32_t* token_out;
    const float* logits;       // top_k 1..64: the logits, penalised as they are read (no copy)
    int32_t* host_out;         // optional (mapped host memory): [2..3] the state, then [0] the token
    int32_t* dev_token;        // optional: the token also stored here (a decode step's next input)
    // the full-sort path (top_k 0 or above kSmpKeep, or a large vocabulary):
    // every key sorted by merging 2048-key runs (two buffers of n_sort keys,
    // n_sort = blocks * 2048 rounded up to a power of two), then the
    // reference's arithmetic over the first k of them
    unsigned long long* sort_a;
    unsigned long long* sort_b;
    uint32_t n_sort;
    float* probs;              // [k] e^((l - max) / temperature) of the sorted candidates
};

struct ArgmaxFinishParams {
    const float* part_val;
    const uint32_t* part_idx;
    uint32_t parts;
    int32_t* token_out;
    int32_t* pos;              // if non-null: gen[pos] = token, pos += 1
    int32_t* gen;
    int32_t* host_token;       // optional: the token also stored here (mapped host memory, read after a sync)
    const int* range_flag;     // optional: copied to host_token[1] before the token is stored
};

constexpr int kAttnSub = 32;         // positions staged in LDS at a time
constexpr int kAttnMaxHd = 128;
constexpr int kAttnMaxGroups = 4;
constexpr int kAttnMaxSplits = 64;
// fused short-context attention + o (gemv_q4m_attn_kernel): 32-position
// passes, 8 waves x 4 row slots, at most 8 passes (256 positions)
constexpr int kFusedWaves = 8;
constexpr uint32_t kFusedPass = 32;
constexpr int kFusedMaxPasses = 8;
// chunked step: at most this many column tiles (position chunks) per head,
// and the polls of a workgroup waiting for its head's chunk states before
// it gives up and flags the step (the states of every workgroup of a launch
// are in place within microseconds when the grid is resident at once)
constexpr uint32_t kChunkMaxTiles = 16;
constexpr uint32_t kChunkHeads = 64;
constexpr uint32_t kChunkSpin = 1u << 20;
constexpr uint32_t kChunkCountStride = 32;   // u32 counters 128 bytes apart: [kChunkHeads][32]
constexpr uint32_t kChunkCountWords = kChunkHeads * kChunkCountStride / 2;   // as int64 words

struct AttnParams {
    const float* q;            // kernel-level: q [H*hd] fp32, already rotated
    const long long* qkv_acc;  // model: fixed-point q|k|v; RoPE + cache append here
    const float* ss_in;        // model: partial sums of squares of the q|k|v GEMV input
    uint32_t ss_n;             // (the RMSNorm factor is applied to q, k, v here)
    uint32_t norm_n;
    const float* rope_cos;
    const float* rope_sin;
    int use_rope;
    uint32_t half;
    void* kc;                  // [capacity][KVH][hd]
    void* vc;
    int kv_f16;
    const int32_t* pos;        // L = *pos + 1 when non-null
    uint32_t L;
    uint32_t H, KVH, hd, groups;
    float scale;               // 1 / sqrt(hd)
    uint32_t chunk;            // positions per split (multiple of kAttnSub); 0: attn_chunk_for(L)
    float* part;               // [KVH][s_max][groups][hd + 2]
    uint32_t s_max;
    uint32_t nsg;              // 1: attn_decode_kernel; > 1: attn_decode_long_kernel (4 passes in flight per split)
    // cache addressing: element (pos, kvh, d) at pos * kv_ps + kvh * kv_hs + d;
    // kv_ps = 0: token-major [pos][KVH][hd] (kv_ps = KVH hd, kv_hs = hd)
    uint64_t kv_ps, kv_hs;
};

// o projection with the attention of its query head computed in the
// prologue (gemv_q4m_attn_kernel): the GEMV part (K slice = one head) and
// the model-mode attention inputs (q|k|v sums, RoPE tables, cache).
struct AttnOParams {
    GemvParams g;
    AttnParams a;
    // chunked step (gemv_q4m_attn_kernel with CH): workgroup (head h, column
    // tile j) attends over positions [32 NP j, 32 NP (j + 1)) and leaves its
    // state (acc[hd], m, l) in a.part at [h][j]; ch_count[h * 32] counts the
    // states in place. The counters are zero when the launch starts (the
    // next launch that clears this accumulator region clears them again).
    uint32_t* ch_count;
    uint32_t ch_spin;          // polls before a workgroup gives up waiting (kChunkSpin)
};

struct AttnCombineParams {
    const float* part;
    const int32_t* pos;
    uint32_t L, H, KVH, hd, groups, chunk, s_max;
    float* out;                // [H * hd]
};

struct EmbedParams {
    const uint8_t* w;        // Q4 packed or F16 words
    const uint16_t* scales;  // Q4 only
    int fmt;                 // 1 = Q4, 0 = F16
    uint32_t hidden;
    uint32_t vocab;          // token ids are clamped to [0, vocab)
    const int32_t* tok_src;
    const int32_t* tok_idx;  // optional index into tok_src (prefill: position)
    long long* xacc;         // fixed-point residual stream, set (not added)
};

}  // namespace qora
