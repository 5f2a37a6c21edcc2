/*
 * qora_hip.h - C ABI of the MI355X (gfx950) batch-1 decode path for QORA's
 * SmolLM3-3B engine. This is the drop-in boundary a host (the reference's
 * Rust crate through an FFI shim, or C/C++/Python) links against.
 *
 * Conventions (mirroring the reference, src/gemv.rs):
 *  - Every function returns an int status: 0 = OK, negative = error; no
 *    exception or panic crosses the ABI. qora_hip_last_error() describes the
 *    last failure on a context. Shape misuse, which panics in the reference
 *    (slice indexing, debug_assert! at gemv.rs:598), returns
 *    QORA_HIP_E_INVALID here.
 *  - Host buffers passed in are borrowed for the duration of the call and
 *    copied; outputs go to caller-allocated buffers (the reference returns
 *    fresh Vec<f32>).
 *  - A context owns its device memory, one HIP stream and the captured decode
 *    graphs. It is NOT thread-safe: one host thread per context, like the
 *    reference's single decode thread (gpu_inference.rs:523-533).
 *  - Weight layouts are exactly the reference's (gemv.rs:23-38, 29-38):
 *    Q4: packed[k][n/2] u8 (byte = q[2i] | q[2i+1] << 4, value (q-8)*scale),
 *        scales[k][n/32] IEEE binary16; F16: data[k][n] binary16. k is the
 *    input dim, n the output dim; the tied embedding is k = vocab, n = hidden.
 */
#ifndef QORA_HIP_H
#define QORA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QORA_HIP_OK 0
#define QORA_HIP_E_INVALID (-1) /* bad argument or shape */
#define QORA_HIP_E_DEVICE (-2)  /* HIP runtime failure / no device */
#define QORA_HIP_E_NOMEM (-3)   /* device allocation failed */
#define QORA_HIP_E_STATE (-4)   /* wrong call order: no model, cache full ... */
#define QORA_HIP_E_IO (-5)      /* .qora file read/parse failure */
/* A decode step's fixed-point values left their range: a residual value of
 * 2^25 or more, or one projection term of 2^20 or more (the reference's fp32
 * would go on). The step's results are not valid; steps are refused until
 * qora_hip_kv_reset, qora_hip_prefill or qora_hip_kv_upload. */
#define QORA_HIP_E_RANGE (-6)

typedef struct qora_hip_ctx qora_hip_ctx;

/* ---- context ------------------------------------------------------------
 * Replaces the device set-up of generate_gpu (gpu_inference.rs:512-591): the
 * 256 MB VRAM probe and backend init become one call that fails with an
 * error code, so the host keeps the reference's "any Err falls back to CPU"
 * behaviour (main.rs:143-151). QORA_HIP_FORCE_FAIL=init makes it fail on
 * purpose (host-side fault injection for fallback tests). */
int qora_hip_create(int device, qora_hip_ctx** out);
int qora_hip_destroy(qora_hip_ctx* ctx);
const char* qora_hip_last_error(const qora_hip_ctx* ctx);
/* Number of compute units of the context's device. */
int qora_hip_device_cus(const qora_hip_ctx* ctx);

/* ---- weights -------------------------------------------------------------
 * Upload one matrix in the reference layout (WeightRef::Q4 / ::F16,
 * gemv.rs:67-70; load_weight in gpu_loader.rs:51-131). Returns a weight id.
 * packed_len must be k*n/2, n_scales k*n/32, n a multiple of 32. */
int qora_hip_upload_q4(qora_hip_ctx* ctx, const uint8_t* packed, size_t packed_len,
                       const uint16_t* scales_f16, size_t n_scales, uint64_t k, uint64_t n,
                       uint32_t* wid);
int qora_hip_upload_f16(qora_hip_ctx* ctx, const uint16_t* w, size_t len, uint64_t k, uint64_t n,
                        uint32_t* wid);
/* Device addresses of an uploaded weight (scales is NULL for F16). */
int qora_hip_weight_ptrs(qora_hip_ctx* ctx, uint32_t wid, void** packed_or_data, void** scales);
/* Frees an uploaded weight (dropping a WeightData, gemv.rs:99-102; the id is
 * not reused). Refused with QORA_HIP_E_STATE while the initialised model
 * uses it. */
int qora_hip_release_weight(qora_hip_ctx* ctx, uint32_t wid);

/* ---- model ---------------------------------------------------------------
 * DecodeWeights::from_parts (gemv.rs:306-337) + the per-layer config of
 * LayerWeightData (gemv.rs:105-119). Norm vectors and RoPE tables are host
 * pointers (copied); the projection weights are ids from the upload calls,
 * in the order q, k, v, o, gate, up, down per layer. */
typedef struct {
    uint32_t num_layers, vocab, hidden, intermediate;
    uint32_t num_heads, num_kv_heads, head_dim, num_kv_groups, rope_half_dim;
    uint32_t format;                        /* 0 = F16, 1 = Q4 (save.rs:198-202) */
    const uint32_t* layer_wids;             /* [num_layers*7] */
    const uint16_t* const* input_norm;      /* [num_layers] -> f16[hidden] */
    const uint16_t* const* post_attn_norm;  /* [num_layers] -> f16[hidden] */
    uint32_t embed_wid;                     /* k = vocab, n = hidden */
    const uint16_t* final_norm;             /* f16[hidden] */
    const float* rope_cos;                  /* [rope_positions][rope_half_dim] */
    const float* rope_sin;
    uint64_t rope_positions;
    const uint8_t* use_rope;                /* [num_layers]: the file's no_rope_layers (1 = rotate) */
    uint32_t kv_capacity;                   /* positions held on device; 0 = the RoPE table length
                                               (65536 without RoPE layers), every position the
                                               model can place */
    uint32_t kv_dtype;                      /* 0 = f32 (reference RawKvCache), 1 = f16 */
} qora_model_desc;

/* The KV cache starts zero-filled; QORA_HIP_KV_FILL=nan fills it with NaN
 * bit patterns instead (a test that slots past the current length never
 * reach the attention output). */
int qora_hip_model_init(qora_hip_ctx* ctx, const qora_model_desc* desc);

/* save::load_model (save.rs:154-210): read a .qora v1 file, upload it and
 * initialise the model in one call. */
int qora_hip_load_model(qora_hip_ctx* ctx, const char* path, uint32_t kv_capacity, uint32_t kv_dtype);

/* raw_prefill (gemv.rs:1027-1190): the cache is reset, the n prompt tokens
 * are run, and the last token's logits (optional, caller buffer [vocab]) and
 * greedy token (optional) are returned. */
int qora_hip_prefill(qora_hip_ctx* ctx, const uint32_t* ids, size_t n, float* logits_or_null,
                     uint32_t* argmax_or_null);

/* forward_decode_raw (gemv.rs:872-1019) + the greedy branch of
 * sample_token_top_k (generate.rs:346-352): one token at the current cache
 * position. The KV cache lives on the device inside ctx. */
int qora_hip_decode(qora_hip_ctx* ctx, uint32_t token, float* logits_or_null, uint32_t* argmax_or_null);

/* The greedy decode loop of generate_raw (generate.rs:308-322) with
 * temperature 0, without EOS or loop-detection stops: feeds `token`, then
 * each argmax back, `steps` times, on the device; tokens_out[i] is the
 * argmax of step i. */
int qora_hip_generate_greedy(qora_hip_ctx* ctx, uint32_t token, uint32_t steps, uint32_t* tokens_out);

/* Sampling settings of generate_raw (GenerateParams, generate.rs:15-35;
 * defaults main.rs:130-141). */
typedef struct {
    float temperature;          /* <= 0: greedy, the first-max rule */
    float top_p;                /* nucleus mass, e.g. 0.95 */
    uint32_t top_k;             /* candidates kept (the reference default is 20); 0 = the whole
                                   vocabulary, as sample_token_top_k (generate.rs:357-363) */
    float repetition_penalty;   /* <= 1: off; once per occurrence in the last 64 history tokens */
    float presence_penalty;     /* <= 0: off; once for every token present in the history */
} qora_sample_params;

/* apply_repetition_penalty, then apply_presence_penalty, then
 * sample_token_top_k (generate.rs:64-91, 345-395) on device logits [vocab]
 * (vocab <= 4194304; the logits are not modified). top_k 1..64 on a
 * vocabulary of up to 131072 takes the fast path (each block's best 64);
 * any other top_k sorts every logit on the device. The penalties apply only
 * when temperature > 0, as at every call site (generate.rs:141-145, 216-235).
 * history is the host array
 * of generated tokens, rng_state the Rng (xorshift64, generate.rs:38-61)
 * state, advanced in place by the one draw a sampled token takes. The
 * reference seeds it from the clock; callers pass any non-zero seed. */
int qora_hip_sample(qora_hip_ctx* ctx, const float* logits, uint64_t vocab, const uint32_t* history,
                    uint64_t n_history, const qora_sample_params* params, uint64_t* rng_state, uint32_t* token,
                    void* stream);

/* qora_hip_decode followed by qora_hip_sample on the step's logits, which
 * stay on the device (copied out only if logits_or_null is given). The
 * sampled token is also left on the device as the next step's input, so a
 * following qora_hip_decode / qora_hip_decode_sample with that token uploads
 * nothing. */
int qora_hip_decode_sample(qora_hip_ctx* ctx, uint32_t token, const uint32_t* history, uint64_t n_history,
                           const qora_sample_params* params, uint64_t* rng_state, float* logits_or_null,
                           uint32_t* token_out);

/* Context bound of the fused short-context step (no counterpart in the
 * reference): graph-driven steps that append a position below it run each
 * layer's attention inside the o-projection kernel; longer contexts take the
 * split attention kernel. 0 = never (no model, F16 weights, a shape the fused
 * kernel does not cover, or QORA_HIP_ATTN_O=0 at model_init). */
uint32_t qora_hip_attn_o_limit(const qora_hip_ctx* ctx);

/* Context bound of the chunked step (no counterpart in the reference):
 * graph-driven steps that append a position from qora_hip_attn_o_limit up to
 * below this bound keep attention and the o projection in one kernel, each
 * column-tile workgroup of a head attending over its own chunk of the
 * positions; longer contexts take the split attention kernel. 0 = never (no
 * fused step, a shape or device the chunked kernel does not cover, or
 * QORA_HIP_ATTN_CHUNK=0 at model_init). */
uint32_t qora_hip_attn_chunk_limit(const qora_hip_ctx* ctx);

/* RawKvCache access (gemv.rs:154-166): current length, reset to empty, and a
 * copy of one layer's [len][kv_heads][head_dim] K and V as f32. */
int qora_hip_kv_len(qora_hip_ctx* ctx, uint64_t* len);
int qora_hip_kv_reset(qora_hip_ctx* ctx);
int qora_hip_kv_download(qora_hip_ctx* ctx, uint32_t layer, float* k, float* v);
/* The reverse of kv_download (a caller-built RawKvCache, gemv.rs:154-166):
 * rows [0, len) of one layer's K and V from f32 [len][kv_heads][head_dim]
 * (rounded to binary16 for an f16 cache), and the cache length set to len,
 * so the next decode step appends at position len. Upload every layer with
 * the same len. len <= kv_capacity (and the RoPE table length). */
int qora_hip_kv_upload(qora_hip_ctx* ctx, uint32_t layer, const float* k, const float* v, uint64_t len);

/* ---- device memory and graphs (harness plumbing) ------------------------ */
int qora_hip_malloc(qora_hip_ctx* ctx, size_t bytes, void** dptr);
int qora_hip_free(qora_hip_ctx* ctx, void* dptr);
int qora_hip_memcpy_h2d(qora_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int qora_hip_memcpy_d2h(qora_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int qora_hip_synchronize(qora_hip_ctx* ctx);
/* The context's hipStream_t, as void*. */
void* qora_hip_stream(qora_hip_ctx* ctx);
/* Capture the kernel-level calls issued between begin and end on the
 * context stream into a graph; replay it `count` times. */
int qora_hip_capture_begin(qora_hip_ctx* ctx);
int qora_hip_capture_end(qora_hip_ctx* ctx, void** graph_exec);
int qora_hip_graph_launch(qora_hip_ctx* ctx, void* graph_exec, uint32_t count);
int qora_hip_graph_destroy(qora_hip_ctx* ctx, void* graph_exec);

/* ---- kernel-level entry points ------------------------------------------
 * Device pointers, launched on `stream` (a hipStream_t; NULL = the context
 * stream). Scratch for split-K partials comes from the context. */

/* gemv -> gemv_q4 (gemv.rs:382-387, 646-675; simd.rs:44-83): y = x . W,
 * W Q4 [k][n] in the projection layout. */
int qora_hip_gemv_q4(qora_hip_ctx* ctx, const void* packed, const void* scales, const float* x, float* y,
                     uint64_t k, uint64_t n, void* stream);
/* No counterpart in the reference: qora_hip_gemv_q4 for callers that cannot
 * allocate device memory (code under stream capture, tight serving loops,
 * harnesses that forbid hipMalloc). It calls no hipMalloc, hipFree or other
 * allocating routine: its fixed-point accumulator is a static device array
 * of 65536 int64 words (512 KiB per device, held until the process ends), so
 * n is limited to 65536 (larger n returns QORA_HIP_E_INVALID). Same kernels
 * and results as qora_hip_gemv_q4. Every call on a device shares that
 * device's array: calls that overlap on one device (two streams, two
 * contexts) race. */
int qora_hip_gemv_q4_noalloc(qora_hip_ctx* ctx, const void* packed, const void* scales, const float* x, float* y,
                             uint64_t k, uint64_t n, void* stream);
/* gemv_f16 (gemv.rs:534-567; simd.rs:151-176). */
int qora_hip_gemv_f16(qora_hip_ctx* ctx, const void* w, const float* x, float* y, uint64_t k, uint64_t n,
                      void* stream);
/* Single-launch forms of the two GEMVs above, used inside the decode step:
 * acc[j] += (x . W)[j] as fixed point (int64, value = acc / 2^36), so the
 * split-K partial sums land in any order with identical results. gate_up
 * accumulates gate into acc[0:n] and up into acc[n:2n]. acc_to_f32 converts
 * (paired: y = silu(acc[0:n]) * acc[n:2n], the epilogue of gemv.rs:494-500). */
int qora_hip_gemv_q4_accumulate(qora_hip_ctx* ctx, const void* packed, const void* scales, const float* x,
                                long long* acc, uint64_t k, uint64_t n, void* stream);
int qora_hip_gate_up_q4_accumulate(qora_hip_ctx* ctx, const void* gate_packed, const void* gate_scales,
                                   const void* up_packed, const void* up_scales, const float* x, long long* acc,
                                   uint64_t k, uint64_t n, void* stream);
int qora_hip_acc_to_f32(qora_hip_ctx* ctx, const long long* acc, uint64_t n, int paired, float* y, void* stream);
/* The decode step's GEMV on uploaded weights (same kernel, plain fp32 x):
 * prepare packs weight `wid` (paired != 0: the gate|up pair wid, wid_up)
 * once into the tile layout the decode step streams (each workgroup reads
 * one contiguous block); run launches acc[j] += (x . W)[j] exactly like
 * the *_accumulate calls above; release frees the packed copy. prepare and
 * release allocate / free, so they are refused during capture. */
int qora_hip_gemv_prepare(qora_hip_ctx* ctx, uint32_t wid, uint32_t wid_up, int paired, uint32_t* gemv_id);
int qora_hip_gemv_run(qora_hip_ctx* ctx, uint32_t gemv_id, const float* x, long long* acc, void* stream);
int qora_hip_gemv_release(qora_hip_ctx* ctx, uint32_t gemv_id);
/* The decode step's lm_head on an uploaded Q4 weight [rows][cols] (the tied
 * embedding; lm_head_parallel_q4, gemv.rs:825-864, with the greedy branch
 * of sample_token_top_k, generate.rs:346-352): prepare packs it once into
 * the matrix-core tile layout (cols must be 128, 256, 512, 1024 or 2048);
 * run writes logits[r] = sum_c x[c] W[r][c] and, if argmax_device is not
 * NULL, the first-max index as a device int32. Release the id with
 * qora_hip_gemv_release. */
int qora_hip_lm_head_prepare(qora_hip_ctx* ctx, uint32_t wid, uint32_t* lm_id);
int qora_hip_lm_head_run(qora_hip_ctx* ctx, uint32_t lm_id, const float* x, float* logits, int32_t* argmax_device,
                         void* stream);
/* lm_head_parallel_q4 / _f16 (gemv.rs:797-864): y[r] = sum_c x[c] W[r][c]
 * over a [rows][cols] matrix (the tied embedding); cols/32 must divide 64. */
int qora_hip_gemv_q4_rowdot(qora_hip_ctx* ctx, const void* packed, const void* scales, const float* x,
                            float* y, uint64_t rows, uint64_t cols, void* stream);
int qora_hip_gemv_f16_rowdot(qora_hip_ctx* ctx, const void* w, const float* x, float* y, uint64_t rows,
                             uint64_t cols, void* stream);
/* fused_gate_up_gemv (gemv.rs:392-502; simd.rs:87-147):
 * out = silu(x . Wg) * (x . Wu). */
int qora_hip_gate_up_q4(qora_hip_ctx* ctx, const void* gate_packed, const void* gate_scales,
                        const void* up_packed, const void* up_scales, const float* x, float* out,
                        uint64_t k, uint64_t n, void* stream);
int qora_hip_gate_up_f16(qora_hip_ctx* ctx, const void* gate_w, const void* up_w, const float* x, float* out,
                         uint64_t k, uint64_t n, void* stream);
/* embed_lookup_q4 (gemv.rs:710-736) over the whole matrix: out [k][n] f32. */
int qora_hip_dequant_q4(qora_hip_ctx* ctx, const void* packed, const void* scales, uint64_t k, uint64_t n,
                        float* out, void* stream);
/* rms_norm_f16 (gemv.rs:744-753), eps 1e-6. */
int qora_hip_rmsnorm(qora_hip_ctx* ctx, const float* x, const void* gamma, uint64_t n, float* out, void* stream);
/* apply_rope_raw (gemv.rs:757-778), in place on [num_heads][head_dim]. */
int qora_hip_rope(qora_hip_ctx* ctx, float* data, uint32_t num_heads, uint32_t head_dim, const float* cos_t,
                  const float* sin_t, uint32_t half_dim, uint32_t position, void* stream);
/* Decode attention of forward_decode_raw (gemv.rs:914-989): q [H*hd],
 * caches token-major [L][KVH][hd] (f32, or f16 when kv_f16), out [H*hd]. */
int qora_hip_attn_decode(qora_hip_ctx* ctx, const float* q, const void* kc, const void* vc, int kv_f16,
                         uint32_t L, uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_dim, float* out,
                         void* stream);
/* gemm -> gemm_q4 / gemm_f16 (gemv.rs:505-511, 569-588, 677-706), the
 * prefill projection: y [T][n] = x [T][k] . W for uploaded weight `wid`
 * (k a multiple of 32), on the matrix cores with both operands split into two
 * binary16 parts (the batched-prefill GEMM). Scratch comes from the context. */
int qora_hip_gemm(qora_hip_ctx* ctx, uint32_t wid, const float* x, float* y, uint64_t T, void* stream);
/* Causal attention of raw_prefill (gemv.rs:1088-1130) for T query rows at
 * positions pos0 .. pos0 + T - 1: q [T][H*hd] (already rotated), caches
 * token-major [pos0 + T][KVH][hd] (f32, or f16 when kv_f16), out [T][H*hd];
 * row t attends to cache rows 0 .. pos0 + t. */
int qora_hip_attn_prefill(qora_hip_ctx* ctx, const float* q, const void* kc, const void* vc, int kv_f16,
                          uint32_t pos0, uint32_t T, uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_dim,
                          float* out, void* stream);
/* Greedy branch of sample_token_top_k (generate.rs:346-352); the token is
 * written to a device int32. */
int qora_hip_argmax(qora_hip_ctx* ctx, const float* logits, uint64_t n, int32_t* out_device, void* stream);

/* ---- synthetic inputs (host only; no device needed) ----------------------
 * Seeded, counter-based generator (splitmix64 streams keyed by seed and
 * tensor id) for the benchmark configurations. The reference has no
 * quantizer (gemv.rs:168-170 is empty); these produce bytes in its layout.
 *   q4  : v = U{-7..7}, stored q = v + 8; scale = f16(|z| * 0.02 / 7)
 *   f16 : f16(z * std)
 *   f32 : z
 * z is a Box-Muller normal draw from two 32-bit uniforms, with ln and cos
 * evaluated from correctly rounded float64 operations (exactly reproducible). */
void qora_synth_q4(uint64_t seed, uint64_t tensor_id, uint64_t k, uint64_t n, uint8_t* packed,
                   uint16_t* scales);
void qora_synth_f16(uint64_t seed, uint64_t tensor_id, uint64_t count, float stddev, uint16_t* out);
void qora_synth_f32(uint64_t seed, uint64_t tensor_id, uint64_t count, float* out);
void qora_synth_tokens(uint64_t seed, uint64_t tensor_id, uint64_t count, uint32_t vocab, uint32_t* out);
/* cos/sin(pos * theta^(-2i/(2*half_dim))) in float64, rounded to f32;
 * [positions][half_dim]. The reference reads these tables from the file
 * (save.rs:195-196) and has no generator. */
void qora_rope_tables(uint64_t positions, uint32_t half_dim, double theta, float* cos_out, float* sin_out);

/* ---- .qora v1 files (save.rs) -------------------------------------------- */
/* save_model (save.rs:119-151) from host buffers laid out like
 * qora_model_desc, with host weight pointers instead of ids:
 * w_data[l*7+j] / w_scales[l*7+j] (scales NULL for F16). */
typedef struct {
    uint32_t num_layers, vocab, hidden, intermediate;
    uint32_t num_heads, num_kv_heads, head_dim, num_kv_groups, rope_half_dim;
    uint32_t format;
    const void* const* w_data;
    const uint16_t* const* w_scales;
    const uint16_t* const* input_norm;
    const uint16_t* const* post_attn_norm;
    const void* embed_data;
    const uint16_t* embed_scales;
    const uint16_t* final_norm;
    const float* rope_cos;
    const float* rope_sin;
    uint64_t rope_positions;
    const uint8_t* use_rope;
} qora_host_model;
int qora_file_write(const char* path, const qora_host_model* m);

#ifdef __cplusplus
}
#endif
#endif /* QORA_HIP_H */
