// Launch-parameter structs shared by the kernels and the host launch code.
#pragma once

#include <stdint.h>

namespace qora {

enum WFmt : int { FMT_F16 = 0, FMT_Q4 = 1 };
enum Epi : int { EPI_STORE = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_QKV = 3 };

struct GemvSeg {
    const uint8_t* w;         // Q4 packed bytes or F16 words (as bytes)
    const uint16_t* scales;   // Q4 only
    uint32_t groups;          // n / 32
    uint32_t tile0;           // first column tile (concatenated mode)
    uint32_t tiles;           // column tiles of this segment
};

struct GemvParams {
    GemvSeg seg[3];
    int nseg;
    int paired;               // 1: seg0 = gate, seg1 = up, lanes split in halves
    const float* x;           // input vector [k]
    const uint16_t* gamma;    // optional RMSNorm gamma [k] (prologue)
    uint32_t k;
    uint32_t tiles;           // total column tiles
    uint32_t splits;          // S
    uint32_t rows_per_split;  // KR
    float* partials;          // [S][tiles][GT*32]
    uint32_t* counters;       // [tiles], zero between launches
    int epi;
    float* y;                 // STORE / RESID / SILU destination
    // QKV epilogue
    float* q_out;
    void* kcache;
    void* vcache;
    int kv_f16;
    uint32_t head_dim, half_dim, kv_stride;
    const float* rope_cos;
    const float* rope_sin;
    const int32_t* pos;
    int use_rope;
};

struct RowdotParams {
    const uint8_t* w;
    const uint16_t* scales;
    uint32_t rows, cols;       // cols = hidden, multiple of 32, cols/32 divides 64
    const float* x;
    const uint16_t* gamma;     // optional RMSNorm prologue
    float* y;                  // [rows]
    int do_argmax;
    float* part_val;           // [gridDim.x]
    uint32_t* part_idx;
    uint32_t* counter;         // zero between launches
    int32_t* token_out;        // argmax result
    int32_t* pos;              // if non-null: gen[pos] = argmax, pos += 1
    int32_t* gen;
};

constexpr int kAttnChunk = 32;
constexpr int kAttnMaxHd = 128;
constexpr int kAttnMaxGroups = 4;

struct AttnParams {
    const float* q;          // [H * hd]
    const void* kc;
    const void* vc;
    int kv_f16;
    const int32_t* pos;      // L = *pos + 1 when non-null
    uint32_t L;              // used when pos is null
    uint32_t H, KVH, hd, groups;
    float scale;             // 1 / sqrt(hd)
    float* part;             // [KVH][s_max][groups][hd + 2]
    uint32_t* counters;      // [KVH], zero between launches
    uint32_t s_max;
    float* out;              // [H * hd]
};

struct EmbedParams {
    const uint8_t* w;        // Q4 packed or F16 words
    const uint16_t* scales;  // Q4 only
    int fmt;                 // 1 = Q4, 0 = F16
    uint32_t hidden;
    uint32_t vocab;          // token ids are clamped to [0, vocab)
    const int32_t* tok_src;
    const int32_t* tok_idx;  // optional index into tok_src (prefill: position)
    float* x;
};

}  // namespace qora
