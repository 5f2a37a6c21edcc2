/*
 * CPU oracle for the QORA SmolLM3-3B batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * CPU algorithm (Rust crate `qora`, files src/gemv.rs and src/simd.rs). It is
 * the checker that the HIP kernels are compared against, and the timed CPU
 * baseline in bench.py. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function names the reference lines it restates. Summation orders,
 * the skip-on-zero branches, the k-split into T partial vectors and the
 * order in which partials are added follow the reference exactly, so with
 * the same T the oracle reproduces the reference's floating-point result
 * (the reference's own result depends on rayon's thread count T).
 *
 * Pin of each exported function (tests/test_oracle.py unless named):
 *   oq_h2f                  all 65536 codes vs IEEE widening (numpy)
 *   oq_dequant_q4(_row)     all 256 bytes x every scale class vs float64;
 *                           one-hot GEMV rows
 *   oq_gemv_q4_rows         numpy float32 restatement of the row order
 *   oq_gemv_q4              single pass and k-split (T = 1, 3, 12) bit-exact
 *                           vs numpy float32 restatements; exact-arithmetic
 *                           regime = float64; one-hot, zero, linearity
 *   oq_fused_gate_up_q4     partials bit-exact vs restatement, SiLU vs float64
 *   oq_gemv_f16             scalar order bit-exact (numpy float32); AVX-512
 *                           order, single pass and k-split (T = 3, 12 at
 *                           k*n >= 4e6), bit-exact vs an FMA restatement that
 *                           is itself checked against libm fmaf
 *   oq_fused_gate_up_f16    two GEMVs + SiLU vs float64
 *   oq_lm_head_q4 / _f16    row-dot order bit-exact (numpy float32)
 *   oq_rms_norm_f16         order bit-exact; constant-vector closed form
 *   oq_apply_rope           identity at pos 0, pair norms, float64
 *   oq_softmax              uniform scores, float64
 *   oq_attention_decode     L = 1, identical keys, GQA mapping, float64
 *   oq_argmax               first-max rules (ties, NaN, +-inf)
 *   oq_forward_decode /     float64 restatement of the model (tests/
 *   oq_prefill              model_f64.py), Q4 and F16 (both F16 dispatch
 *                           orders, T = 1 and 3); greedy chain; F16 embedding
 *                           row exact
 *   oq_kv_*                 caches vs the float64 model's; kv_set resumes
 *                           bit-identically
 *   oq_set_threads          results identical for 1 and 4 threads
 *   oq_rng_next_f32,        tests/test_sampling.py: integer xorshift
 *   penalties, top-k        restatement, penalty semantics, one-draw cases,
 *                           sampled frequencies vs the float64 distribution
 * Parity unpinned (no reference test or import can pin it): the exact
 * bits of libm expf used in SiLU and softmax (glibc expf here vs the Rust
 * platform libm there), covered by tolerance only; the reference's rayon
 * thread count T, taken as a parameter.
 */
#ifndef QORA_ORACLE_H
#define QORA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 -> binary32 widening (half 2.7.1 f16::to_f32). Exact. */
float oq_h2f(uint16_t h);

/* ---- kernels (src/gemv.rs, src/simd.rs) ---- */

/* embed_lookup_q4 (gemv.rs:710-736): dequantize row `row` of a Q4 matrix. */
void oq_dequant_q4_row(const uint8_t* packed, const uint16_t* scales,
                       uint64_t n, uint64_t row, float* out);
/* Full-matrix dequant (same arithmetic as embed_lookup_q4, all rows). */
void oq_dequant_q4(const uint8_t* packed, const uint16_t* scales,
                   uint64_t k, uint64_t n, float* out);

/* gemv_q4_inner (gemv.rs:596-641) / simd::gemv_q4_avx512 (simd.rs:44-83):
 * rows [k0, k1) of the outer-product LUT accumulation into out[n]. */
void oq_gemv_q4_rows(const float* x, const uint8_t* packed, const uint16_t* scales,
                     uint64_t n, uint64_t k0, uint64_t k1, float* out);

/* gemv_q4 (gemv.rs:646-675): k*n < 4e6 -> one pass; else T partials. */
void oq_gemv_q4(const float* x, const uint8_t* packed, const uint16_t* scales,
                uint64_t k, uint64_t n, int T, float* out);

/* fused_gate_up_q4 (gemv.rs:412-502): always T partials, then SiLU * up. */
void oq_fused_gate_up_q4(const float* x,
                         const uint8_t* gp, const uint16_t* gs,
                         const uint8_t* up, const uint16_t* us,
                         uint64_t k, uint64_t n, int T, float* out);

/* gemv_f16 (gemv.rs:534-567). avx512 != 0 follows the AVX-512 branch
 * (FMA per element, k-split into T partials when k*n >= 4e6,
 * simd.rs:151-176); avx512 == 0 follows the scalar branch (mul then add,
 * one sequential pass). */
void oq_gemv_f16(const float* x, const uint16_t* w, uint64_t k, uint64_t n,
                 int T, int avx512, float* out);

/* fused_gate_up_gemv F16 fallback (gemv.rs:395-407). */
void oq_fused_gate_up_f16(const float* x, const uint16_t* gw, const uint16_t* uw,
                          uint64_t k, uint64_t n, int T, int avx512, float* out);

/* lm_head_parallel_q4 (gemv.rs:825-864): row-dot over [vocab][hidden]. */
void oq_lm_head_q4(const float* x, const uint8_t* packed, const uint16_t* scales,
                   uint64_t vocab, uint64_t hidden, float* out);
/* lm_head_parallel_f16 (gemv.rs:805-822). */
void oq_lm_head_f16(const float* x, const uint16_t* w, uint64_t vocab,
                    uint64_t hidden, float* out);

/* rms_norm_f16 (gemv.rs:744-753), eps hard-coded 1e-6. */
void oq_rms_norm_f16(const float* x, const uint16_t* gamma, uint64_t size, float* out);

/* apply_rope_raw (gemv.rs:757-778), in place. */
void oq_apply_rope(float* data, uint64_t num_heads, uint64_t head_dim,
                   const float* cos_t, const float* sin_t, uint64_t half_dim,
                   uint64_t position);

/* softmax_raw (gemv.rs:782-793), in place. */
void oq_softmax(float* scores, uint64_t n);

/* Decode attention of forward_decode_raw (gemv.rs:914-989): q [H*hd],
 * caches token-major [L][KVH][hd] f32, out [H*hd]. */
void oq_attention_decode(const float* q, const float* kc, const float* vc,
                         uint64_t L, uint64_t num_heads, uint64_t num_kv_heads,
                         uint64_t head_dim, float* out);

/* Greedy branch of sample_token_top_k (generate.rs:346-352): first max. */
uint32_t oq_argmax(const float* logits, uint64_t n);

/* ---- model (gemv.rs:172-338, 866-1190) ---- */

typedef struct {
    uint32_t num_layers, vocab, hidden, intermediate;
    uint32_t num_heads, num_kv_heads, head_dim, num_kv_groups, rope_half_dim;
    uint32_t format;                 /* 0 = F16, 1 = Q4 (save.rs:198-202) */
    /* per layer, 7 weights in order q,k,v,o,gate,up,down:
     * Q4: w_data = packed bytes, w_scales = f16 scales;
     * F16: w_data = f16 words, w_scales = NULL. */
    const void* const* w_data;       /* [num_layers*7] */
    const uint16_t* const* w_scales; /* [num_layers*7] */
    const uint16_t* const* in_norm;  /* [num_layers] f16[hidden] */
    const uint16_t* const* post_norm;/* [num_layers] f16[hidden] */
    const void* embed_data;          /* [vocab][hidden] */
    const uint16_t* embed_scales;    /* Q4 only */
    const uint16_t* final_norm;      /* f16[hidden] */
    const float* rope_cos;           /* [positions][half_dim] */
    const float* rope_sin;
    const uint8_t* use_rope;         /* [num_layers], the file's no_rope_layers */
} oq_model_desc;

/* RawKvCache (gemv.rs:154-166): per layer token-major f32 K and V. */
typedef struct oq_kv oq_kv;
oq_kv* oq_kv_create(uint32_t num_layers, uint32_t kv_stride, uint64_t capacity);
void oq_kv_free(oq_kv* kv);
uint64_t oq_kv_len(const oq_kv* kv, uint32_t layer);
const float* oq_kv_k(const oq_kv* kv, uint32_t layer);
const float* oq_kv_v(const oq_kv* kv, uint32_t layer);
int oq_kv_set(oq_kv* kv, uint32_t layer, const float* k, const float* v, uint64_t len);

/* sampling (generate.rs:38-91, 345-395) */
float oq_rng_next_f32(uint64_t* state);
void oq_repetition_penalty(float* logits, uint64_t vocab, const uint32_t* gen, uint64_t n, float penalty);
void oq_presence_penalty(float* logits, uint64_t vocab, const uint32_t* gen, uint64_t n, float penalty);
uint32_t oq_sample_top_k(const float* logits, uint64_t vocab, float temperature, float top_p, uint64_t top_k,
                         uint64_t* rng);


/* forward_decode_raw (gemv.rs:872-1019). T = rayon thread count. Returns 0
 * on success, -1 if the cache is full. logits: [vocab]. */
int oq_forward_decode(const oq_model_desc* m, oq_kv* kv, uint32_t token,
                      int T, int avx512, float* logits);

/* raw_prefill (gemv.rs:1027-1190). kv must be empty. logits: [vocab] of the
 * last token. Returns 0, or -1 on bad input. */
int oq_prefill(const oq_model_desc* m, oq_kv* kv, const uint32_t* ids, uint64_t n,
               int T, float* logits);

/* Number of OpenMP threads used for the independent work items (attention
 * heads, lm_head chunks, k-split partials); does not change any result. */
void oq_set_threads(int nthreads);

#ifdef __cplusplus
}
#endif
#endif
