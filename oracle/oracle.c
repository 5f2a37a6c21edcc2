/*
 * CPU oracle for the QORA SmolLM3-3B batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY: a restatement of the reference CPU algorithm
 * (Rust crate `qora`: src/gemv.rs, src/simd.rs, src/generate.rs) used as the
 * checker for the HIP library and as the timed CPU baseline. The product
 * library never links or calls this file. The header oracle.h lists what
 * pins each function and which parts are "parity unpinned".
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp). Floating
 * point contraction is off so every `a * b + c` the reference writes as a
 * separate multiply and add stays two roundings; the one place the
 * reference fuses (the AVX-512 F16 GEMV, simd.rs:166) calls fmaf.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>
#include <immintrin.h>

/* ------------------------------------------------------------------ */
/* binary16 <-> binary32                                               */
/* ------------------------------------------------------------------ */

static float g_h2f_table[65536];
static int g_tables_ready = 0;
static int g_nthreads = 0;
static int g_has_avx512 = -1;

static float h2f_slow(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { mant <<= 1; ++e; } while ((mant & 0x400u) == 0);
            mant &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void init_tables(void) {
    if (g_tables_ready) return;
#pragma omp critical(oq_tables)
    {
        if (!g_tables_ready) {
            for (uint32_t i = 0; i < 65536; ++i) g_h2f_table[i] = h2f_slow((uint16_t)i);
            g_has_avx512 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("fma") &&
                           __builtin_cpu_supports("f16c");
            __atomic_store_n(&g_tables_ready, 1, __ATOMIC_RELEASE);
        }
    }
}

#define H2F(h) (g_h2f_table[(uint16_t)(h)])

float oq_h2f(uint16_t h) { init_tables(); return H2F(h); }


void oq_set_threads(int nthreads) { g_nthreads = nthreads; }

static int nthreads(void) { return g_nthreads > 0 ? g_nthreads : omp_get_max_threads(); }

/* ------------------------------------------------------------------ */
/* Q4 dequant: embed_lookup_q4 (gemv.rs:710-736)                       */
/* ------------------------------------------------------------------ */

void oq_dequant_q4_row(const uint8_t* packed, const uint16_t* scales, uint64_t n,
                       uint64_t row, float* out) {
    init_tables();
    const uint64_t G = n / 32;
    const uint8_t* p = packed + row * G * 16;
    const uint16_t* s = scales + row * G;
    for (uint64_t g = 0; g < G; ++g) {
        const float scale = H2F(s[g]);
        for (int j = 0; j < 16; ++j) {
            const uint8_t b = p[g * 16 + j];
            const int q0 = (int)(b & 0x0F) - 8;
            const int q1 = (int)((b >> 4) & 0x0F) - 8;
            out[g * 32 + 2 * j] = scale * (float)q0;
            out[g * 32 + 2 * j + 1] = scale * (float)q1;
        }
    }
}

void oq_dequant_q4(const uint8_t* packed, const uint16_t* scales, uint64_t k, uint64_t n,
                   float* out) {
    init_tables();
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int64_t r = 0; r < (int64_t)k; ++r) oq_dequant_q4_row(packed, scales, n, (uint64_t)r, out + r * n);
}

/* ------------------------------------------------------------------ */
/* Q4 GEMV rows: gemv_q4_inner (gemv.rs:596-641) and its AVX-512 twin   */
/* simd::gemv_q4_avx512 (simd.rs:44-83). The two are bit-identical: both */
/* add fl(s * (q-8)) per element, row by row, group by group, with      */
/* s = f32(scale) * x[row]. The AVX form below computes s*(q-8) with a  */
/* vector multiply instead of a LUT permute; the products are the same. */
/* ------------------------------------------------------------------ */

static inline void q4_group_generic(float* o, const uint8_t* p, float s) {
    for (int j = 0; j < 16; ++j) {
        const uint8_t b = p[j];
        o[2 * j] += s * (float)((int)(b & 15) - 8);
        o[2 * j + 1] += s * (float)((int)(b >> 4) - 8);
    }
}

__attribute__((target("avx512f")))
static inline void q4_group_avx512(float* o, const uint8_t* p, float s) {
    const __m512i idx_a = _mm512_setr_epi32(0, 16, 1, 17, 2, 18, 3, 19, 4, 20, 5, 21, 6, 22, 7, 23);
    const __m512i idx_b = _mm512_setr_epi32(8, 24, 9, 25, 10, 26, 11, 27, 12, 28, 13, 29, 14, 30, 15, 31);
    const __m512i b32 = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i*)p));
    const __m512i eight = _mm512_set1_epi32(8);
    const __m512 lo = _mm512_cvtepi32_ps(_mm512_sub_epi32(_mm512_and_si512(b32, _mm512_set1_epi32(15)), eight));
    const __m512 hi = _mm512_cvtepi32_ps(_mm512_sub_epi32(_mm512_srli_epi32(b32, 4), eight));
    const __m512 sv = _mm512_set1_ps(s);
    const __m512 lo_v = _mm512_mul_ps(lo, sv);
    const __m512 hi_v = _mm512_mul_ps(hi, sv);
    const __m512 c0 = _mm512_permutex2var_ps(lo_v, idx_a, hi_v); /* columns 0..15 */
    const __m512 c1 = _mm512_permutex2var_ps(lo_v, idx_b, hi_v); /* columns 16..31 */
    _mm512_storeu_ps(o, _mm512_add_ps(_mm512_loadu_ps(o), c0));
    _mm512_storeu_ps(o + 16, _mm512_add_ps(_mm512_loadu_ps(o + 16), c1));
}

__attribute__((target("avx512f")))
static void q4_rows_avx512(const float* x, const uint8_t* packed, const uint16_t* scales,
                           uint64_t n, uint64_t k0, uint64_t k1, float* out) {
    const uint64_t G = n / 32;
    for (uint64_t ki = k0; ki < k1; ++ki) {
        const float v = x[ki];
        if (v == 0.0f) continue;
        const uint16_t* srow = scales + ki * G;
        const uint8_t* prow = packed + ki * G * 16;
        for (uint64_t g = 0; g < G; ++g) {
            const float s = H2F(srow[g]) * v;
            if (s == 0.0f) continue;
            q4_group_avx512(out + g * 32, prow + g * 16, s);
        }
    }
}

static void q4_rows_generic(const float* x, const uint8_t* packed, const uint16_t* scales,
                            uint64_t n, uint64_t k0, uint64_t k1, float* out) {
    const uint64_t G = n / 32;
    for (uint64_t ki = k0; ki < k1; ++ki) {
        const float v = x[ki];
        if (v == 0.0f) continue;
        const uint16_t* srow = scales + ki * G;
        const uint8_t* prow = packed + ki * G * 16;
        for (uint64_t g = 0; g < G; ++g) {
            const float s = H2F(srow[g]) * v;
            if (s == 0.0f) continue;
            q4_group_generic(out + g * 32, prow + g * 16, s);
        }
    }
}

void oq_gemv_q4_rows(const float* x, const uint8_t* packed, const uint16_t* scales,
                     uint64_t n, uint64_t k0, uint64_t k1, float* out) {
    init_tables();
    memset(out, 0, n * sizeof(float));
    if (g_has_avx512) q4_rows_avx512(x, packed, scales, n, k0, k1, out);
    else q4_rows_generic(x, packed, scales, n, k0, k1, out);
}

/* Sum T partial vectors in thread order starting from zeros
 * (gemv.rs:668-673, 485-492). */
static void sum_partials(const float* partials, const int* valid, int T, uint64_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    for (int t = 0; t < T; ++t) {
        if (!valid[t]) continue;
        const float* p = partials + (uint64_t)t * n;
        for (uint64_t j = 0; j < n; ++j) out[j] += p[j];
    }
}

void oq_gemv_q4(const float* x, const uint8_t* packed, const uint16_t* scales,
                uint64_t k, uint64_t n, int T, float* out) {
    init_tables();
    if (k * n < 4000000ull || T <= 1) {
        /* T == 1: one chunk [0, k) summed onto zeros, identical to one pass. */
        oq_gemv_q4_rows(x, packed, scales, n, 0, k, out);
        return;
    }
    const uint64_t chunk = (k + (uint64_t)T - 1) / (uint64_t)T;
    float* partials = (float*)malloc((uint64_t)T * n * sizeof(float));
    int* valid = (int*)calloc((size_t)T, sizeof(int));
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int t = 0; t < T; ++t) {
        const uint64_t ks = (uint64_t)t * chunk;
        const uint64_t ke = ((uint64_t)(t + 1) * chunk < k) ? (uint64_t)(t + 1) * chunk : k;
        if (ks >= k) continue;
        valid[t] = 1;
        oq_gemv_q4_rows(x, packed, scales, n, ks, ke, partials + (uint64_t)t * n);
    }
    sum_partials(partials, valid, T, n, out);
    free(partials);
    free(valid);
}

/* SiLU * up (gemv.rs:494-500 and 401-405). */
static void silu_mul(const float* gate, const float* up, uint64_t n, float* out) {
    for (uint64_t j = 0; j < n; ++j) {
        const float g = gate[j];
        const float silu_g = g / (1.0f + expf(-g));
        out[j] = silu_g * up[j];
    }
}

/* fused_gate_up_q4 (gemv.rs:412-502) / simd::fused_gate_up_q4_avx512
 * (simd.rs:87-147): one pass over x, k-split into T partials always. */
void oq_fused_gate_up_q4(const float* x, const uint8_t* gp, const uint16_t* gs,
                         const uint8_t* up, const uint16_t* us, uint64_t k, uint64_t n,
                         int T, float* out) {
    init_tables();
    if (T < 1) T = 1;
    const uint64_t G = n / 32;
    const uint64_t chunk = (k + (uint64_t)T - 1) / (uint64_t)T;
    float* pg = (float*)calloc((uint64_t)T * n, sizeof(float));
    float* pu = (float*)calloc((uint64_t)T * n, sizeof(float));
    int* valid = (int*)calloc((size_t)T, sizeof(int));
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int t = 0; t < T; ++t) {
        const uint64_t ks = (uint64_t)t * chunk;
        const uint64_t ke = ((uint64_t)(t + 1) * chunk < k) ? (uint64_t)(t + 1) * chunk : k;
        if (ks >= k) continue;
        valid[t] = 1;
        float* og = pg + (uint64_t)t * n;
        float* ou = pu + (uint64_t)t * n;
        for (uint64_t ki = ks; ki < ke; ++ki) {
            const float v = x[ki];
            if (v == 0.0f) continue;
            for (uint64_t g = 0; g < G; ++g) {
                const float sg = H2F(gs[ki * G + g]) * v;
                const float su = H2F(us[ki * G + g]) * v;
                if (sg == 0.0f && su == 0.0f) continue;
                if (g_has_avx512) {
                    if (sg != 0.0f) q4_group_avx512(og + g * 32, gp + (ki * G + g) * 16, sg);
                    if (su != 0.0f) q4_group_avx512(ou + g * 32, up + (ki * G + g) * 16, su);
                } else {
                    if (sg != 0.0f) q4_group_generic(og + g * 32, gp + (ki * G + g) * 16, sg);
                    if (su != 0.0f) q4_group_generic(ou + g * 32, up + (ki * G + g) * 16, su);
                }
            }
        }
    }
    float* gate = (float*)malloc(n * sizeof(float));
    float* upv = (float*)malloc(n * sizeof(float));
    sum_partials(pg, valid, T, n, gate);
    sum_partials(pu, valid, T, n, upv);
    silu_mul(gate, upv, n, out);
    free(gate); free(upv); free(pg); free(pu); free(valid);
}

/* ------------------------------------------------------------------ */
/* F16 GEMV: gemv_f16 (gemv.rs:534-567), simd::gemv_f16_avx512         */
/* (simd.rs:151-176).                                                   */
/* ------------------------------------------------------------------ */

__attribute__((target("avx512f,fma,f16c")))
static void f16_rows_avx512(const float* x, const uint16_t* w, uint64_t k, uint64_t n, float* out) {
    /* simd.rs:151-176: per row skip x == 0; 16-wide cvtph + FMA; the
     * n % 16 tail is a scalar multiply then add. */
    memset(out, 0, n * sizeof(float));
    const uint64_t n16 = n / 16 * 16;
    for (uint64_t ki = 0; ki < k; ++ki) {
        const float v = x[ki];
        if (v == 0.0f) continue;
        const __m512 vv = _mm512_set1_ps(v);
        const uint16_t* row = w + ki * n;
        uint64_t j = 0;
        for (; j < n16; j += 16) {
            const __m512 wf = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(row + j)));
            _mm512_storeu_ps(out + j, _mm512_fmadd_ps(vv, wf, _mm512_loadu_ps(out + j)));
        }
        for (; j < n; ++j) out[j] += v * H2F(row[j]);
    }
}

static void f16_rows_fma_generic(const float* x, const uint16_t* w, uint64_t k, uint64_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    const uint64_t n16 = n / 16 * 16;
    for (uint64_t ki = 0; ki < k; ++ki) {
        const float v = x[ki];
        if (v == 0.0f) continue;
        const uint16_t* row = w + ki * n;
        uint64_t j = 0;
        for (; j < n16; ++j) out[j] = fmaf(v, H2F(row[j]), out[j]);
        for (; j < n; ++j) out[j] += v * H2F(row[j]);
    }
}

static void f16_rows_fma(const float* x, const uint16_t* w, uint64_t k, uint64_t n, float* out) {
    if (g_has_avx512) f16_rows_avx512(x, w, k, n, out);
    else f16_rows_fma_generic(x, w, k, n, out);
}

void oq_gemv_f16(const float* x, const uint16_t* w, uint64_t k, uint64_t n, int T, int avx512,
                 float* out) {
    init_tables();
    if (!avx512) {
        /* gemv.rs:558-566: scalar multiply then add, no skip, one pass. */
        memset(out, 0, n * sizeof(float));
        for (uint64_t ki = 0; ki < k; ++ki) {
            const float v = x[ki];
            const uint16_t* row = w + ki * n;
            for (uint64_t j = 0; j < n; ++j) out[j] += v * H2F(row[j]);
        }
        return;
    }
    if (k * n < 4000000ull || T <= 1) {
        f16_rows_fma(x, w, k, n, out);
        return;
    }
    const uint64_t chunk = (k + (uint64_t)T - 1) / (uint64_t)T;
    float* partials = (float*)malloc((uint64_t)T * n * sizeof(float));
    int* valid = (int*)calloc((size_t)T, sizeof(int));
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (int t = 0; t < T; ++t) {
        const uint64_t ks = (uint64_t)t * chunk;
        const uint64_t ke = ((uint64_t)(t + 1) * chunk < k) ? (uint64_t)(t + 1) * chunk : k;
        if (ks >= k) continue;
        valid[t] = 1;
        f16_rows_fma(x + ks, w + ks * n, ke - ks, n, partials + (uint64_t)t * n);
    }
    sum_partials(partials, valid, T, n, out);
    free(partials);
    free(valid);
}

void oq_fused_gate_up_f16(const float* x, const uint16_t* gw, const uint16_t* uw, uint64_t k,
                          uint64_t n, int T, int avx512, float* out) {
    float* gate = (float*)malloc(n * sizeof(float));
    float* upv = (float*)malloc(n * sizeof(float));
    oq_gemv_f16(x, gw, k, n, T, avx512, gate);
    oq_gemv_f16(x, uw, k, n, T, avx512, upv);
    silu_mul(gate, upv, n, out);
    free(gate);
    free(upv);
}

/* ------------------------------------------------------------------ */
/* lm_head (gemv.rs:805-864): sequential dot per vocabulary row.        */
/* ------------------------------------------------------------------ */

void oq_lm_head_q4(const float* x, const uint8_t* packed, const uint16_t* scales,
                   uint64_t vocab, uint64_t hidden, float* out) {
    init_tables();
    const uint64_t G = hidden / 32;
#pragma omp parallel for schedule(static, 256) num_threads(nthreads())
    for (int64_t v = 0; v < (int64_t)vocab; ++v) {
        float dot = 0.0f;
        for (uint64_t g = 0; g < G; ++g) {
            const float scale = H2F(scales[(uint64_t)v * G + g]);
            if (scale == 0.0f) continue;
            float lut[16];
            for (int q = 0; q < 16; ++q) lut[q] = (q == 8) ? 0.0f : scale * (float)(q - 8);
            const uint8_t* p = packed + ((uint64_t)v * G + g) * 16;
            const float* xi = x + g * 32;
            for (int j = 0; j < 16; ++j) {
                const uint8_t b = p[j];
                dot += xi[2 * j] * lut[b & 0x0F];
                dot += xi[2 * j + 1] * lut[b >> 4];
            }
        }
        out[v] = dot;
    }
}

void oq_lm_head_f16(const float* x, const uint16_t* w, uint64_t vocab, uint64_t hidden,
                    float* out) {
    init_tables();
#pragma omp parallel for schedule(static, 256) num_threads(nthreads())
    for (int64_t v = 0; v < (int64_t)vocab; ++v) {
        const uint16_t* row = w + (uint64_t)v * hidden;
        float sum = 0.0f;
        for (uint64_t j = 0; j < hidden; ++j) sum += x[j] * H2F(row[j]);
        out[v] = sum;
    }
}

/* ------------------------------------------------------------------ */
/* RMSNorm, RoPE, softmax, attention, argmax                            */
/* ------------------------------------------------------------------ */

void oq_rms_norm_f16(const float* x, const uint16_t* gamma, uint64_t size, float* out) {
    init_tables();
    float sum_sq = 0.0f;
    for (uint64_t i = 0; i < size; ++i) sum_sq += x[i] * x[i];
    const float inv_rms = 1.0f / sqrtf(sum_sq / (float)size + 1e-6f);
    for (uint64_t i = 0; i < size; ++i) out[i] = x[i] * inv_rms * H2F(gamma[i]);
}

void oq_apply_rope(float* data, uint64_t num_heads, uint64_t head_dim, const float* cos_t,
                   const float* sin_t, uint64_t half_dim, uint64_t position) {
    const uint64_t off = position * half_dim;
    for (uint64_t h = 0; h < num_heads; ++h) {
        float* d = data + h * head_dim;
        for (uint64_t i = 0; i < half_dim; ++i) {
            const float x1 = d[i];
            const float x2 = d[half_dim + i];
            const float c = cos_t[off + i];
            const float s = sin_t[off + i];
            d[i] = x1 * c - x2 * s;
            d[half_dim + i] = x2 * c + x1 * s;
        }
    }
}

void oq_softmax(float* scores, uint64_t n) {
    float max_val = -INFINITY;
    for (uint64_t i = 0; i < n; ++i) max_val = fmaxf(max_val, scores[i]);
    float sum = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        scores[i] = expf(scores[i] - max_val);
        sum += scores[i];
    }
    const float inv_sum = 1.0f / sum;
    for (uint64_t i = 0; i < n; ++i) scores[i] *= inv_sum;
}

static void attention_head(const float* q, const float* kc, const float* vc, uint64_t L,
                           uint64_t kv_stride, uint64_t kvh, uint64_t head_dim, float scale,
                           float* scores, float* out) {
    for (uint64_t s = 0; s < L; ++s) {
        const float* kv = kc + s * kv_stride + kvh * head_dim;
        float dot = 0.0f;
        for (uint64_t d = 0; d < head_dim; ++d) dot += q[d] * kv[d];
        scores[s] = dot * scale;
    }
    oq_softmax(scores, L);
    for (uint64_t d = 0; d < head_dim; ++d) out[d] = 0.0f;
    for (uint64_t s = 0; s < L; ++s) {
        const float* vv = vc + s * kv_stride + kvh * head_dim;
        const float p = scores[s];
        for (uint64_t d = 0; d < head_dim; ++d) out[d] += p * vv[d];
    }
}

void oq_attention_decode(const float* q, const float* kc, const float* vc, uint64_t L,
                         uint64_t num_heads, uint64_t num_kv_heads, uint64_t head_dim, float* out) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    const uint64_t groups = num_heads / num_kv_heads;
    const uint64_t kv_stride = num_kv_heads * head_dim;
#pragma omp parallel num_threads(nthreads())
    {
        float* scores = (float*)malloc((L ? L : 1) * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t h = 0; h < (int64_t)num_heads; ++h)
            attention_head(q + h * head_dim, kc, vc, L, kv_stride, (uint64_t)h / groups, head_dim,
                           scale, scores, out + h * head_dim);
        free(scores);
    }
}

uint32_t oq_argmax(const float* logits, uint64_t n) {
    uint64_t max_idx = 0;
    float max_val = -INFINITY;
    for (uint64_t i = 0; i < n; ++i) {
        if (logits[i] > max_val) { max_val = logits[i]; max_idx = i; }
    }
    return (uint32_t)max_idx;
}

/* ------------------------------------------------------------------ */
/* Model: forward_decode_raw (gemv.rs:872-1019), raw_prefill            */
/* (gemv.rs:1027-1190).                                                 */
/* ------------------------------------------------------------------ */

struct oq_kv {
    uint32_t num_layers, kv_stride;
    uint64_t capacity;
    float** k;
    float** v;
    uint64_t* len;
};

oq_kv* oq_kv_create(uint32_t num_layers, uint32_t kv_stride, uint64_t capacity) {
    oq_kv* kv = (oq_kv*)calloc(1, sizeof(oq_kv));
    kv->num_layers = num_layers;
    kv->kv_stride = kv_stride;
    kv->capacity = capacity;
    kv->k = (float**)calloc(num_layers, sizeof(float*));
    kv->v = (float**)calloc(num_layers, sizeof(float*));
    kv->len = (uint64_t*)calloc(num_layers, sizeof(uint64_t));
    for (uint32_t i = 0; i < num_layers; ++i) {
        kv->k[i] = (float*)calloc(capacity * kv_stride, sizeof(float));
        kv->v[i] = (float*)calloc(capacity * kv_stride, sizeof(float));
    }
    return kv;
}

void oq_kv_free(oq_kv* kv) {
    if (!kv) return;
    for (uint32_t i = 0; i < kv->num_layers; ++i) { free(kv->k[i]); free(kv->v[i]); }
    free(kv->k); free(kv->v); free(kv->len); free(kv);
}

uint64_t oq_kv_len(const oq_kv* kv, uint32_t layer) { return kv->len[layer]; }
const float* oq_kv_k(const oq_kv* kv, uint32_t layer) { return kv->k[layer]; }
const float* oq_kv_v(const oq_kv* kv, uint32_t layer) { return kv->v[layer]; }

/* A caller-built RawKvCache entry (gemv.rs:154-166): rows [0, len) of one
 * layer, token-major [len][kv_stride]. */
int oq_kv_set(oq_kv* kv, uint32_t layer, const float* k, const float* v, uint64_t len) {
    if (layer >= kv->num_layers || len > kv->capacity) return -1;
    /* copied in 1 MiB pieces on every thread: the first write to fresh cache
     * pages is what costs, and the threads take those page faults in parallel */
    const uint64_t total = len * kv->kv_stride, piece = 1u << 18;
    const int64_t pieces = (int64_t)((total + piece - 1) / piece);
#pragma omp parallel for schedule(dynamic, 4) num_threads(nthreads())
    for (int64_t i = 0; i < 2 * pieces; ++i) {
        const uint64_t at = (uint64_t)(i % pieces) * piece;
        const uint64_t cnt = total - at < piece ? total - at : piece;
        if (i < pieces) memcpy(kv->k[layer] + at, k + at, cnt * sizeof(float));
        else memcpy(kv->v[layer] + at, v + at, cnt * sizeof(float));
    }
    kv->len[layer] = len;
    return 0;
}

enum { W_Q = 0, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN };

typedef struct { uint64_t k, n; } shape_t;

static shape_t weight_shape(const oq_model_desc* m, int w) {
    const uint64_t H = m->hidden, I = m->intermediate;
    const uint64_t qd = (uint64_t)m->num_heads * m->head_dim;
    const uint64_t kvd = (uint64_t)m->num_kv_heads * m->head_dim;
    shape_t s;
    switch (w) {
    case W_Q: s.k = H; s.n = qd; break;
    case W_K: case W_V: s.k = H; s.n = kvd; break;
    case W_O: s.k = qd; s.n = H; break;
    case W_GATE: case W_UP: s.k = H; s.n = I; break;
    default: s.k = I; s.n = H; break;
    }
    return s;
}

/* gemv dispatch (gemv.rs:382-387). */
static void model_gemv(const oq_model_desc* m, uint32_t layer, int w, const float* x, int T,
                       int avx512, float* out) {
    const shape_t s = weight_shape(m, w);
    const uint64_t idx = (uint64_t)layer * 7 + (uint64_t)w;
    if (m->format == 1)
        oq_gemv_q4(x, (const uint8_t*)m->w_data[idx], m->w_scales[idx], s.k, s.n, T, out);
    else
        oq_gemv_f16(x, (const uint16_t*)m->w_data[idx], s.k, s.n, T, avx512, out);
}

/* gemm (gemv.rs:506-511, 571-588, 680-706): every token row is one
 * sequential pass over all k rows; the F16 variant is the scalar
 * multiply-then-add loop. */
static void model_gemm_row(const oq_model_desc* m, uint32_t layer, int w, const float* x,
                           float* out) {
    const shape_t s = weight_shape(m, w);
    const uint64_t idx = (uint64_t)layer * 7 + (uint64_t)w;
    if (m->format == 1) {
        oq_gemv_q4_rows(x, (const uint8_t*)m->w_data[idx], m->w_scales[idx], s.n, 0, s.k, out);
    } else {
        const uint16_t* wd = (const uint16_t*)m->w_data[idx];
        memset(out, 0, s.n * sizeof(float));
        for (uint64_t ki = 0; ki < s.k; ++ki) {
            const float v = x[ki];
            for (uint64_t j = 0; j < s.n; ++j) out[j] += v * H2F(wd[ki * s.n + j]);
        }
    }
}

/* embed_lookup (gemv.rs:515-526). */
static void model_embed(const oq_model_desc* m, uint32_t token, float* out) {
    const uint64_t H = m->hidden;
    if (m->format == 1) {
        oq_dequant_q4_row((const uint8_t*)m->embed_data, m->embed_scales, H, token, out);
    } else {
        const uint16_t* e = (const uint16_t*)m->embed_data + (uint64_t)token * H;
        for (uint64_t j = 0; j < H; ++j) out[j] = H2F(e[j]);
    }
}

static void model_lm_head(const oq_model_desc* m, const float* x, float* logits) {
    if (m->format == 1)
        oq_lm_head_q4(x, (const uint8_t*)m->embed_data, m->embed_scales, m->vocab, m->hidden, logits);
    else
        oq_lm_head_f16(x, (const uint16_t*)m->embed_data, m->vocab, m->hidden, logits);
}

int oq_forward_decode(const oq_model_desc* m, oq_kv* kv, uint32_t token, int T, int avx512,
                      float* logits) {
    init_tables();
    const uint64_t H = m->hidden, I = m->intermediate;
    const uint64_t hd = m->head_dim, nh = m->num_heads, nkv = m->num_kv_heads;
    const uint64_t qd = nh * hd, kvd = nkv * hd;
    if (token >= m->vocab) return -1;
    float* x = (float*)malloc(H * 4);
    float* xn = (float*)malloc(H * 4);
    float* q = (float*)malloc(qd * 4);
    float* kn = (float*)malloc(kvd * 4);
    float* vn = (float*)malloc(kvd * 4);
    float* attn = (float*)malloc(qd * 4);
    float* o = (float*)malloc(H * 4);
    float* inter = (float*)malloc(I * 4);
    int rc = 0;
    model_embed(m, token, x);
    for (uint32_t i = 0; i < m->num_layers && rc == 0; ++i) {
        const uint64_t off = kv->len[i];
        if (off >= kv->capacity) { rc = -1; break; }
        oq_rms_norm_f16(x, m->in_norm[i], H, xn);
        model_gemv(m, i, W_Q, xn, T, avx512, q);
        model_gemv(m, i, W_K, xn, T, avx512, kn);
        model_gemv(m, i, W_V, xn, T, avx512, vn);
        if (m->use_rope[i]) {
            oq_apply_rope(q, nh, hd, m->rope_cos, m->rope_sin, m->rope_half_dim, off);
            oq_apply_rope(kn, nkv, hd, m->rope_cos, m->rope_sin, m->rope_half_dim, off);
        }
        memcpy(kv->k[i] + off * kvd, kn, kvd * 4);
        memcpy(kv->v[i] + off * kvd, vn, kvd * 4);
        kv->len[i] = off + 1;
        /* head -> kv head uses num_kv_groups (gemv.rs:923) */
        {
            const float scale = 1.0f / sqrtf((float)hd);
            const uint64_t L = off + 1;
#pragma omp parallel num_threads(nthreads())
            {
                float* scores = (float*)malloc(L * sizeof(float));
#pragma omp for schedule(static)
                for (int64_t h = 0; h < (int64_t)nh; ++h)
                    attention_head(q + h * hd, kv->k[i], kv->v[i], L, kvd,
                                   (uint64_t)h / m->num_kv_groups, hd, scale, scores, attn + h * hd);
                free(scores);
            }
        }
        model_gemv(m, i, W_O, attn, T, avx512, o);
        for (uint64_t j = 0; j < H; ++j) x[j] += o[j];
        oq_rms_norm_f16(x, m->post_norm[i], H, xn);
        {
            const uint64_t ig = (uint64_t)i * 7;
            if (m->format == 1)
                oq_fused_gate_up_q4(xn, (const uint8_t*)m->w_data[ig + W_GATE], m->w_scales[ig + W_GATE],
                                    (const uint8_t*)m->w_data[ig + W_UP], m->w_scales[ig + W_UP], H, I, T,
                                    inter);
            else
                oq_fused_gate_up_f16(xn, (const uint16_t*)m->w_data[ig + W_GATE],
                                     (const uint16_t*)m->w_data[ig + W_UP], H, I, T, avx512, inter);
        }
        model_gemv(m, i, W_DOWN, inter, T, avx512, o);
        for (uint64_t j = 0; j < H; ++j) x[j] += o[j];
    }
    if (rc == 0) {
        oq_rms_norm_f16(x, m->final_norm, H, xn);
        model_lm_head(m, xn, logits);
    }
    free(x); free(xn); free(q); free(kn); free(vn); free(attn); free(o); free(inter);
    return rc;
}

int oq_prefill(const oq_model_desc* m, oq_kv* kv, const uint32_t* ids, uint64_t n, int T,
               float* logits) {
    (void)T; /* prefill GEMMs never k-split (gemv.rs:684-705) */
    init_tables();
    if (n == 0 || n > kv->capacity) return -1;
    for (uint32_t i = 0; i < m->num_layers; ++i)
        if (kv->len[i] != 0) return -1;
    for (uint64_t t = 0; t < n; ++t)
        if (ids[t] >= m->vocab) return -1;
    const uint64_t H = m->hidden, I = m->intermediate;
    const uint64_t hd = m->head_dim, nh = m->num_heads, nkv = m->num_kv_heads;
    const uint64_t qd = nh * hd, kvd = nkv * hd;
    float* x = (float*)malloc(n * H * 4);
    float* xn = (float*)malloc(n * H * 4);
    float* qa = (float*)malloc(n * qd * 4);
    float* attn = (float*)malloc(n * qd * 4);
    float* o = (float*)malloc(n * H * 4);
    float* gate = (float*)malloc(n * I * 4);
    float* upv = (float*)malloc(n * I * 4);
    for (uint64_t t = 0; t < n; ++t) model_embed(m, ids[t], x + t * H);
    for (uint32_t i = 0; i < m->num_layers; ++i) {
        float* ka = kv->k[i];
        float* va = kv->v[i];
#pragma omp parallel for schedule(static) num_threads(nthreads())
        for (int64_t t = 0; t < (int64_t)n; ++t) {
            oq_rms_norm_f16(x + t * H, m->in_norm[i], H, xn + t * H);
            model_gemm_row(m, i, W_Q, xn + t * H, qa + t * qd);
            model_gemm_row(m, i, W_K, xn + t * H, ka + t * kvd);
            model_gemm_row(m, i, W_V, xn + t * H, va + t * kvd);
            if (m->use_rope[i]) {
                oq_apply_rope(qa + t * qd, nh, hd, m->rope_cos, m->rope_sin, m->rope_half_dim, (uint64_t)t);
                oq_apply_rope(ka + t * kvd, nkv, hd, m->rope_cos, m->rope_sin, m->rope_half_dim, (uint64_t)t);
            }
        }
        kv->len[i] = n;
        {
            const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel num_threads(nthreads())
            {
                float* scores = (float*)malloc(n * sizeof(float));
#pragma omp for schedule(static)
                for (int64_t h = 0; h < (int64_t)nh; ++h) {
                    const uint64_t kvh = (uint64_t)h / m->num_kv_groups;
                    for (uint64_t t1 = 0; t1 < n; ++t1)
                        attention_head(qa + t1 * qd + (uint64_t)h * hd, ka, va, t1 + 1, kvd, kvh, hd, scale,
                                       scores, attn + t1 * qd + (uint64_t)h * hd);
                }
                free(scores);
            }
        }
#pragma omp parallel for schedule(static) num_threads(nthreads())
        for (int64_t t = 0; t < (int64_t)n; ++t) {
            model_gemm_row(m, i, W_O, attn + t * qd, o + t * H);
            for (uint64_t j = 0; j < H; ++j) x[t * H + j] += o[t * H + j];
            oq_rms_norm_f16(x + t * H, m->post_norm[i], H, xn + t * H);
            model_gemm_row(m, i, W_GATE, xn + t * H, gate + t * I);
            model_gemm_row(m, i, W_UP, xn + t * H, upv + t * I);
            silu_mul(gate + t * I, upv + t * I, I, gate + t * I);
            model_gemm_row(m, i, W_DOWN, gate + t * I, o + t * H);
            for (uint64_t j = 0; j < H; ++j) x[t * H + j] += o[t * H + j];
        }
    }
    oq_rms_norm_f16(x + (n - 1) * H, m->final_norm, H, xn);
    model_lm_head(m, xn, logits);
    free(x); free(xn); free(qa); free(attn); free(o); free(gate); free(upv);
    return 0;
}


/* ---- sampling (generate.rs:38-91, 345-395) ---- */

/* Rng::next_f32 (generate.rs:54-60): xorshift64 (13, 7, 17), top 24 bits. */
float oq_rng_next_f32(uint64_t* state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (float)(uint32_t)(x >> 40) / 16777216.0f;
}

/* apply_repetition_penalty (generate.rs:64-78): the last min(len, 64) tokens,
 * one penalty per occurrence. */
void oq_repetition_penalty(float* logits, uint64_t vocab, const uint32_t* gen, uint64_t n, float penalty) {
    if (penalty <= 1.0f) return;
    const uint64_t window = n < 64 ? n : 64;
    for (uint64_t i = n - window; i < n; ++i) {
        const uint32_t idx = gen[i];
        if (idx < vocab) {
            if (logits[idx] > 0.0f) logits[idx] /= penalty;
            else logits[idx] *= penalty;
        }
    }
}

/* apply_presence_penalty (generate.rs:80-91): once per distinct token present. */
void oq_presence_penalty(float* logits, uint64_t vocab, const uint32_t* gen, uint64_t n, float penalty) {
    if (penalty <= 0.0f || n == 0) return;
    unsigned char* seen = (unsigned char*)calloc(vocab, 1);
    for (uint64_t i = 0; i < n; ++i)
        if (gen[i] < vocab) seen[gen[i]] = 1;
    for (uint64_t i = 0; i < vocab; ++i)
        if (seen[i]) logits[i] -= penalty;
    free(seen);
}

typedef struct {
    uint32_t id;
    float v;
} oq_cand;

/* sort_by(b.1.partial_cmp(&a.1)) is a stable sort by value descending: equal
 * values keep ascending index order. */
static int oq_cand_cmp(const void* a, const void* b) {
    const oq_cand* x = (const oq_cand*)a;
    const oq_cand* y = (const oq_cand*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

/* sample_token_top_k (generate.rs:345-395). */
uint32_t oq_sample_top_k(const float* logits, uint64_t vocab, float temperature, float top_p, uint64_t top_k,
                         uint64_t* rng) {
    if (temperature <= 0.0f) {
        uint64_t best = 0;
        float bv = -INFINITY;
        for (uint64_t i = 0; i < vocab; ++i)
            if (logits[i] > bv) { bv = logits[i]; best = i; }
        return (uint32_t)best;
    }
    const float inv_temp = 1.0f / temperature;
    float max_logit = -INFINITY;
    for (uint64_t i = 0; i < vocab; ++i) max_logit = fmaxf(max_logit, logits[i]);
    oq_cand* c = (oq_cand*)malloc(vocab * sizeof(oq_cand));
    for (uint64_t i = 0; i < vocab; ++i) { c[i].id = (uint32_t)i; c[i].v = logits[i]; }
    qsort(c, vocab, sizeof(oq_cand), oq_cand_cmp);
    const uint64_t k = top_k > 0 ? (top_k < vocab ? top_k : vocab) : vocab;
    float* p = (float*)malloc(k * sizeof(float));
    float sum = 0.0f;
    for (uint64_t i = 0; i < k; ++i) { p[i] = expf((c[i].v - max_logit) * inv_temp); sum += p[i]; }
    uint32_t out = c[0].id;
    if (sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (uint64_t i = 0; i < k; ++i) p[i] *= inv;
        float cum = 0.0f;
        uint64_t cutoff = k;
        for (uint64_t i = 0; i < k; ++i) {
            cum += p[i];
            if (cum >= top_p) { cutoff = i + 1; break; }
        }
        float total = 0.0f;
        for (uint64_t i = 0; i < cutoff; ++i) total += p[i];
        if (total > 0.0f) {
            const float rand_val = oq_rng_next_f32(rng) * total;
            float acc = 0.0f;
            out = c[0].id;
            for (uint64_t i = 0; i < cutoff; ++i) {
                acc += p[i];
                if (acc >= rand_val) { out = c[i].id; break; }
            }
        }
    }
    free(p);
    free(c);
    return out;
}
