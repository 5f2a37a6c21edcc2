/* The CPU oracle (oracle/oracle.c, test infrastructure) under
 * AddressSanitizer and UndefinedBehaviorSanitizer: every exported function
 * on small, ragged shapes (k and n not multiples of the k-split, 1-row and
 * 1-position cases), a tiny model's prefill and decode steps in Q4 and F16
 * with T = 1 and T = 3 and both F16 orders, the KV cache set/read calls and
 * the sampling functions. The values are checked for being finite; their
 * correctness is pinned by tests/test_oracle.py. Exit status 0 when clean. */
#include "../../oracle/oracle.h"
#include "../../include/qora_hip.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int failures = 0;

static void check_finite(const float* v, size_t n, const char* what) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) {
            fprintf(stderr, "FAIL: %s[%zu] not finite\n", what, i);
            ++failures;
            return;
        }
}

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) abort();
    return p;
}

static void kernels(void) {
    const uint64_t ks[] = {1, 32, 37, 300}, ns[] = {32, 96, 224};
    for (int a = 0; a < 4; ++a)
        for (int b = 0; b < 3; ++b) {
            const uint64_t k = ks[a], n = ns[b];
            uint8_t* p = xmalloc(k * n / 2);
            uint16_t* s = xmalloc(k * n / 32 * 2);
            uint16_t* w = xmalloc(k * n * 2);
            float* x = xmalloc(k * 4);
            float* y = xmalloc(2 * n * 4);
            float* deq = xmalloc(k * n * 4);
            qora_synth_q4(9, k + n, k, n, p, s);
            qora_synth_f16(9, k * n, k * n, 0.02f, w);
            qora_synth_f32(9, 1, k, x);
            for (int T = 1; T <= 12; T += 11) {
                oq_gemv_q4(x, p, s, k, n, T, y);
                check_finite(y, n, "gemv_q4");
                oq_fused_gate_up_q4(x, p, s, p, s, k, n, T, y);
                check_finite(y, n, "gate_up_q4");
                for (int avx = 0; avx < 2; ++avx) {
                    oq_gemv_f16(x, w, k, n, T, avx, y);
                    check_finite(y, n, "gemv_f16");
                    oq_fused_gate_up_f16(x, w, w, k, n, T, avx, y);
                    check_finite(y, n, "gate_up_f16");
                }
            }
            oq_gemv_q4_rows(x, p, s, n, 0, k, y);
            oq_dequant_q4(p, s, k, n, deq);
            oq_dequant_q4_row(p, s, n, k - 1, deq);
            /* row-dot lm_head: k rows of n columns */
            float* xr = xmalloc(n * 4);
            float* yr = xmalloc(k * 4);
            qora_synth_f32(9, 2, n, xr);
            oq_lm_head_q4(xr, p, s, k, n, yr);
            check_finite(yr, k, "lm_head_q4");
            oq_lm_head_f16(xr, w, k, n, yr);
            check_finite(yr, k, "lm_head_f16");
            (void)oq_argmax(yr, k);
            /* RMSNorm of the row's first min(n, k n / 32) values (the scales as gamma) */
            float* zr = xmalloc(n * 4);
            oq_rms_norm_f16(xr, s, n < k * n / 32 ? n : k * n / 32, zr);
            free(xr); free(yr); free(zr);
            free(p); free(s); free(w); free(x); free(y); free(deq);
        }
    /* attention: L = 1, 2, 33 positions, GQA 4 -> 1 and 2 -> 2 */
    for (uint64_t L = 1; L <= 33; L += 16) {
        const uint64_t H = 4, KVH = 1, hd = 32;
        float* q = xmalloc(H * hd * 4);
        float* kc = xmalloc(L * KVH * hd * 4);
        float* vc = xmalloc(L * KVH * hd * 4);
        float* o = xmalloc(H * hd * 4);
        qora_synth_f32(3, 1, H * hd, q);
        qora_synth_f32(3, 2, L * KVH * hd, kc);
        qora_synth_f32(3, 3, L * KVH * hd, vc);
        oq_attention_decode(q, kc, vc, L, H, KVH, hd, o);
        check_finite(o, H * hd, "attention");
        float* ct = xmalloc(8 * 16 * 4);
        float* st = xmalloc(8 * 16 * 4);
        qora_rope_tables(8, 16, 5e6, ct, st);
        oq_apply_rope(q, H, hd, ct, st, 16, 7);
        oq_softmax(q, H * hd);
        check_finite(q, H * hd, "softmax");
        free(ct); free(st); free(q); free(kc); free(vc); free(o);
    }
    /* sampling */
    float logits[100];
    uint32_t gen[70];
    qora_synth_f32(4, 1, 100, logits);
    qora_synth_tokens(4, 2, 70, 120, gen);   /* ids past the vocabulary are skipped */
    oq_repetition_penalty(logits, 100, gen, 70, 1.1f);
    oq_presence_penalty(logits, 100, gen, 70, 1.5f);
    uint64_t rng = 0x9E3779B97F4A7C15ull;
    for (uint64_t top_k = 0; top_k <= 120; top_k += 20) {
        const uint32_t t = oq_sample_top_k(logits, 100, 0.7f, 0.9f, top_k, &rng);
        if (t >= 100) { fprintf(stderr, "FAIL: sample %u\n", t); ++failures; }
    }
    (void)oq_rng_next_f32(&rng);
}

static void model(uint32_t fmt) {
    enum { NL = 2, V = 64, H = 64, I = 96, NH = 2, NKV = 1, HD = 32, HALF = 16, POS = 16 };
    const uint64_t qd = NH * HD, kvd = NKV * HD;
    const uint64_t shapes[7][2] = {{H, qd}, {H, kvd}, {H, kvd}, {qd, H}, {H, I}, {H, I}, {I, H}};
    const void* wd[NL * 7];
    const uint16_t* ws[NL * 7];
    void* owned[NL * 7 * 2 + 8];
    int no = 0;
    for (int l = 0; l < NL; ++l)
        for (int j = 0; j < 7; ++j) {
            const uint64_t k = shapes[j][0], n = shapes[j][1];
            if (fmt == 1) {
                uint8_t* p = xmalloc(k * n / 2);
                uint16_t* s = xmalloc(k * n / 32 * 2);
                qora_synth_q4(7, 16 * l + j, k, n, p, s);
                wd[l * 7 + j] = p;
                ws[l * 7 + j] = s;
                owned[no++] = p;
                owned[no++] = s;
            } else {
                uint16_t* w = xmalloc(k * n * 2);
                qora_synth_f16(7, 16 * l + j, k * n, 0.02f, w);
                wd[l * 7 + j] = w;
                ws[l * 7 + j] = NULL;
                owned[no++] = w;
            }
        }
    uint16_t norms[2 * NL + 1][H];
    for (int i = 0; i < 2 * NL + 1; ++i) qora_synth_f16(8, i, H, 0.5f, norms[i]);
    const uint16_t* in[NL] = {norms[0], norms[2]};
    const uint16_t* post[NL] = {norms[1], norms[3]};
    void* ed;
    uint16_t* es = NULL;
    if (fmt == 1) {
        ed = xmalloc(V * H / 2);
        es = xmalloc(V * H / 32 * 2);
        qora_synth_q4(7, 1000, V, H, ed, es);
    } else {
        ed = xmalloc(V * H * 2);
        qora_synth_f16(7, 1000, V * H, 0.02f, ed);
    }
    owned[no++] = ed;
    if (es) owned[no++] = es;
    float ct[POS * HALF], st[POS * HALF];
    qora_rope_tables(POS, HALF, 5e6, ct, st);
    const uint8_t use_rope[NL] = {0, 1};
    oq_model_desc m = {NL, V, H, I, NH, NKV, HD, NH / NKV, HALF, fmt, wd, ws, in, post, ed, es, norms[2 * NL],
                       ct, st, use_rope};
    const uint32_t ids[5] = {1, 7, 63, 0, 12};
    float logits[V];
    for (int T = 1; T <= 3; T += 2) {
        oq_kv* kv = oq_kv_create(NL, kvd, POS);
        if (oq_prefill(&m, kv, ids, 5, T, logits) != 0) { fprintf(stderr, "FAIL: prefill\n"); ++failures; }
        check_finite(logits, V, "prefill logits");
        for (int s = 0; s < 4; ++s) {
            const int rc = oq_forward_decode(&m, kv, oq_argmax(logits, V), T, s & 1, logits);
            if (rc != 0) { fprintf(stderr, "FAIL: decode %d\n", s); ++failures; }
            check_finite(logits, V, "decode logits");
        }
        /* the cache is full after POS positions: a decode step past it is refused */
        float k1[16 * 32], v1[16 * 32];
        memcpy(k1, oq_kv_k(kv, 1), sizeof k1);
        memcpy(v1, oq_kv_v(kv, 1), sizeof v1);
        if (oq_kv_len(kv, 1) != 9) { fprintf(stderr, "FAIL: kv len\n"); ++failures; }
        if (oq_kv_set(kv, 0, k1, v1, POS) != 0) { fprintf(stderr, "FAIL: kv set\n"); ++failures; }
        if (oq_kv_set(kv, 0, k1, v1, POS + 1) == 0) { fprintf(stderr, "FAIL: kv set past capacity\n"); ++failures; }
        oq_kv_free(kv);
    }
    for (int i = 0; i < no; ++i) free(owned[i]);
}

int main(void) {
    oq_set_threads(3);
    kernels();
    model(1);
    model(0);
    if (failures) {
        fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    printf("oracle_check: clean\n");
    return 0;
}
