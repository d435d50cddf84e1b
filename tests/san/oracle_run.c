/* Test driver (sanitizer tier): every entry point of the CPU oracle
 * (oracle/miattn_oracle.c, q4_oracle.c, prefill_oracle.c, built into this
 * executable with AddressSanitizer and UBSan) on small shapes, including
 * wrapped rings, a slot written twice in one chunk and a negative position.
 * Exits 0 when every output is finite; a sanitizer report aborts the run. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/miattn_oracle.h"
#include "../../oracle/prefill_oracle.h"
#include "../../oracle/q4_oracle.h"

static uint64_t g_state = 0x9e3779b97f4a7c15ull;
static float rnd(void) { /* splitmix64 -> roughly N(0,1) by a sum of uniforms */
    float s = 0.f;
    for (int i = 0; i < 4; ++i) {
        uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        s += (float)(z >> 40) / (float)(1ull << 24) - 0.5f;
    }
    return s * 1.7f;
}
static float *vec(size_t n) {
    float *p = malloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i) p[i] = rnd();
    return p;
}
static int all_finite(const float *p, size_t n, const char *what) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(p[i])) {
            printf("%s: non-finite at %zu\n", what, i);
            return 0;
        }
    return 1;
}
static unsigned char *q4_rows(int rows, int cols) {
    const int nb = cols / 32;
    unsigned char *w = malloc((size_t)rows * nb * 18);
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < nb; ++b) {
            unsigned char *blk = w + ((size_t)r * nb + b) * 18;
            const uint16_t d = ora_f32_to_f16(0.02f + 0.01f * fabsf(rnd()));
            memcpy(blk, &d, 2);
            for (int j = 0; j < 16; ++j) blk[2 + j] = (unsigned char)(rnd() * 97.f);
        }
    return w;
}

int main(void) {
    const int n_layers = 2, n_heads = 8, n_kv = 2, hd = 128, M = 64, kv_dim = n_kv * hd;
    const int dim = n_heads * hd;
    int ok = 1;
    OraKV kv;
    if (ora_kv_alloc(&kv, n_layers, n_kv, hd, M)) return 2;
    for (int l = 0; l < n_layers; ++l)
        for (int s = 0; s < M; ++s) {
            float *k = vec(kv_dim), *v = vec(kv_dim);
            ora_cvt_f32_to_f16(k, ora_kv_k_at(&kv, l, s), kv_dim);
            ora_cvt_f32_to_f16(v, ora_kv_v_at(&kv, l, s), kv_dim);
            free(k);
            free(v);
        }
    kv.len = M;
    float th[64];
    ora_precompute_rope_theta(1e6f, hd, th);
    float *att = malloc(sizeof(float) * n_heads * M), *out = malloc(sizeof(float) * 16 * dim);

    /* decode steps, inside and past the ring */
    for (int pos = 10; pos < 200; pos += 63) {
        float *q = vec(dim), *k = vec(kv_dim), *v = vec(kv_dim);
        ora_decode_step(&kv, 1, q, k, v, pos, th, n_heads, n_kv, att, out);
        ok &= all_finite(out, dim, "decode_step");
        free(q); free(k); free(v);
    }
    /* gqa attention over the ring as it stands */
    {
        float *q = vec(dim);
        ora_gqa_attention(q, att, out, ora_kv_k(&kv, 0), ora_kv_v(&kv, 0), n_heads, n_heads / n_kv,
                          hd, M, 100);
        ok &= all_finite(out, dim, "gqa_attention");
        free(q);
    }
    /* batch: rope, ring write, attention on a wrapped ring */
    {
        const int S = 5, start = 62;
        float *Q = vec((size_t)S * dim), *K = vec((size_t)S * kv_dim), *V = vec((size_t)S * kv_dim);
        ora_apply_rope_batch(Q, K, start, th, n_heads, n_kv, hd, S);
        ora_kv_write_batch(&kv, 0, start, K, V, kv_dim, S);
        ora_attention_batch(Q, out, &kv, 0, start, n_heads, n_kv, hd, S, att);
        ok &= all_finite(out, (size_t)S * dim, "attention_batch");
        free(Q); free(K); free(V);
    }
    /* sequential verify and the chunked prefill's attention */
    {
        const int S = 3;
        float *Q = vec((size_t)S * dim), *K = vec((size_t)S * kv_dim), *V = vec((size_t)S * kv_dim);
        ora_verify_steps(&kv, 1, Q, K, V, 130, S, th, n_heads, n_kv, att, out);
        ok &= all_finite(out, (size_t)S * dim, "verify_steps");
        free(Q); free(K); free(V);
        const int positions[4] = {5, 69, 6, -1};  /* 69 reuses 5's slot; -1 has no window */
        Q = vec((size_t)4 * dim); K = vec((size_t)4 * kv_dim); V = vec((size_t)4 * kv_dim);
        ora_prefill_chunk_attention(&kv, 1, Q, K, V, positions, 4, th, n_heads, n_kv, att, out);
        ok &= all_finite(out, (size_t)4 * dim, "prefill_chunk_attention");
        free(Q); free(K); free(V);
    }
    /* textbook reference and the CPU-baseline drivers */
    {
        const int S = 4;
        float *q = vec((size_t)S * dim), *k = vec((size_t)S * kv_dim), *v = vec((size_t)S * kv_dim);
        ora_ref_gqa_attention(out, q, k, v, S, n_heads, n_kv, hd);
        ok &= all_finite(out, (size_t)S * dim, "ref_gqa_attention");
        free(q); free(k); free(v);
        float *Q = vec((size_t)n_layers * dim), *O = malloc(sizeof(float) * n_layers * 8 * dim);
        ora_decode_layers(Q, O, kv.k_cache, kv.v_cache, n_layers, n_heads, n_heads / n_kv, hd, M,
                          90, 1);
        ok &= all_finite(O, (size_t)n_layers * dim, "decode_layers");
        free(Q);
        Q = vec((size_t)n_layers * 8 * dim);
        ora_attention_batch_layers(Q, O, kv.k_cache, kv.v_cache, n_layers, n_heads, n_kv, hd, M, 60,
                                   8, 1);
        ok &= all_finite(O, (size_t)n_layers * 8 * dim, "attention_batch_layers");
        free(Q); free(O);
    }
    /* Q4_0 x Q8_0 matvecs */
    {
        const int in = 256, rows = 64, kvr = 32;
        float *x = vec(in), *y = malloc(sizeof(float) * rows), *yk = malloc(sizeof(float) * kvr),
              *yv = malloc(sizeof(float) * kvr);
        OraQ8Block q8[256 / ORA_QK];
        ora_quantize_q8_0(x, q8, in);
        unsigned char *W = q4_rows(rows, in), *Wk = q4_rows(kvr, in), *Wv = q4_rows(kvr, in);
        ora_q4_0_q8_0_matvec(W, q8, y, rows, in);
        ok &= all_finite(y, rows, "q4_0_q8_0_matvec");
        ora_q4_0_q8_0_matvec_parallel(W, q8, y, rows, in, 1);
        ora_q4_0_q8_0_matvec_qkv(W, Wk, Wv, q8, y, yk, yv, rows, kvr, in);
        ok &= all_finite(yk, kvr, "matvec_qkv");
        free(x); free(y); free(yk); free(yv); free(W); free(Wk); free(Wv);
    }
    /* the prefill layer: RMSNorm, Q4_0 GEMMs, RoPE, ring write, attention, SwiGLU */
    {
        const int pdim = 256, hidden = 512, ph = 2, pkv = 1, S = 4;
        OraKV pk;
        if (ora_kv_alloc(&pk, 1, pkv, 128, 16)) return 2;
        pk.len = 3;
        OraLayerWeights lw;
        unsigned char *w[7];
        const int shape[7][2] = {{pdim, pdim}, {128, pdim}, {128, pdim}, {pdim, pdim},
                                 {hidden, pdim}, {pdim, hidden}, {hidden, pdim}};
        for (int i = 0; i < 7; ++i) w[i] = q4_rows(shape[i][0], shape[i][1]);
        float *ra = vec(pdim), *rf = vec(pdim), *X = vec((size_t)S * pdim);
        lw.wq = w[0]; lw.wk = w[1]; lw.wv = w[2]; lw.wo = w[3]; lw.w1 = w[4]; lw.w2 = w[5];
        lw.w3 = w[6]; lw.rms_att = ra; lw.rms_ffn = rf;
        ora_prefill_layer(&lw, &pk, X, 0, 14, S, pdim, hidden, ph, pkv, 1e-5f, th, 1);
        ok &= all_finite(X, (size_t)S * pdim, "prefill_layer");
        for (int i = 0; i < 7; ++i) free(w[i]);
        free(ra); free(rf); free(X);
        ora_kv_free(&pk);
    }
    free(att);
    free(out);
    ora_kv_free(&kv);
    printf(ok ? "oracle run: all finite\n" : "oracle run: FAILED\n");
    return ok ? 0 : 1;
}
