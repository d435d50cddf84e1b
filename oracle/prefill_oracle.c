/*
 * prefill_oracle.c -- CPU oracle for the GPU prefill layer (test
 * infrastructure only; see prefill_oracle.h).  Scalar restatement of
 * mistral_ane_prefill.h's BLAS path: vDSP_dotpr / vsmul / vmul / vadd become
 * loops, cblas_sgemm an fp32 triple loop, vvexpf expf.
 */
#include "prefill_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float f16_bits_f32(uint16_t h) { return ora_f16_to_f32(h); }

void ora_rmsnorm_batch(float *out, const float *in, const float *w, int dim, int S, float eps) {
    for (int t = 0; t < S; t++) {
        const float *xi = in + (size_t)t * dim;
        float *xo = out + (size_t)t * dim;
        float ss = 0.0f;
        for (int i = 0; i < dim; i++) ss += xi[i] * xi[i];
        ss = 1.0f / sqrtf(ss / (float)dim + eps);
        for (int i = 0; i < dim; i++) xo[i] = xi[i] * ss;
        for (int i = 0; i < dim; i++) xo[i] = xo[i] * w[i];
    }
}

void ora_dequant_q4_0_rows(const void *W, float *dst, int rows, int cols) {
    const uint8_t *b = (const uint8_t *)W;
    const int bpr = cols / 32;
    for (int r = 0; r < rows; r++) {
        for (int k = 0; k < bpr; k++) {
            const uint8_t *blk = b + ((size_t)r * bpr + k) * 18;
            const float d = f16_bits_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            float *o = dst + (size_t)r * cols + (size_t)k * 32;
            for (int i = 0; i < 16; i++) {
                const uint8_t v = blk[2 + i];
                o[i] = d * ((float)(v & 0x0F) - 8.0f);
                o[i + 16] = d * ((float)(v >> 4) - 8.0f);
            }
        }
    }
}

void ora_q4_0_gemm(const void *W, int out_dim, int in_dim, const float *X, int S, float *Y,
                   int threads) {
    float *w32 = (float *)malloc((size_t)out_dim * in_dim * sizeof(float));
    if (!w32) abort();
    ora_dequant_q4_0_rows(W, w32, out_dim, in_dim);
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads) collapse(2)
#else
    (void)threads;
#endif
    for (int s = 0; s < S; s++) {
        for (int r = 0; r < out_dim; r++) {
            const float *x = X + (size_t)s * in_dim;
            const float *w = w32 + (size_t)r * in_dim;
            float acc = 0.0f;
            for (int k = 0; k < in_dim; k++) acc += x[k] * w[k];
            Y[(size_t)s * out_dim + r] = acc;
        }
    }
    free(w32);
}

void ora_silu_mul(float *gate, const float *up, int n) {
    for (int i = 0; i < n; i++) {
        const float e = expf(-gate[i]);
        const float sig = 1.0f / (1.0f + e);
        gate[i] = (gate[i] * sig) * up[i];
    }
}

void ora_prefill_layer(const OraLayerWeights *lw, OraKV *kv, float *X, int layer, int start_pos,
                       int S, int dim, int hidden, int n_heads, int n_kv_heads, float eps,
                       const float *theta_inv, int threads) {
    const int hd = dim / n_heads;
    const int kv_dim = n_kv_heads * hd;
    const size_t sd = (size_t)S * dim, sk = (size_t)S * kv_dim, sh = (size_t)S * hidden;
    float *Xn = (float *)malloc(sd * sizeof(float));
    float *Q = (float *)malloc(sd * sizeof(float));
    float *K = (float *)malloc(sk * sizeof(float));
    float *V = (float *)malloc(sk * sizeof(float));
    float *A = (float *)malloc(sd * sizeof(float));
    float *G = (float *)malloc(sh * sizeof(float));
    float *U = (float *)malloc(sh * sizeof(float));
    float *att = (float *)malloc((size_t)n_heads * kv->max_seq * sizeof(float));
    if (!Xn || !Q || !K || !V || !A || !G || !U || !att) abort();

    ora_rmsnorm_batch(Xn, X, lw->rms_att, dim, S, eps);
    ora_q4_0_gemm(lw->wq, dim, dim, Xn, S, Q, threads);
    ora_q4_0_gemm(lw->wk, kv_dim, dim, Xn, S, K, threads);
    ora_q4_0_gemm(lw->wv, kv_dim, dim, Xn, S, V, threads);
    ora_apply_rope_batch(Q, K, start_pos, theta_inv, n_heads, n_kv_heads, hd, S);
    ora_kv_write_batch(kv, layer, start_pos, K, V, kv_dim, S);
    ora_attention_batch(Q, A, kv, layer, start_pos, n_heads, n_kv_heads, hd, S, att);
    ora_q4_0_gemm(lw->wo, dim, dim, A, S, Xn, threads);
    for (size_t i = 0; i < sd; i++) X[i] = X[i] + Xn[i];
    ora_rmsnorm_batch(Xn, X, lw->rms_ffn, dim, S, eps);
    ora_q4_0_gemm(lw->w1, hidden, dim, Xn, S, G, threads);
    ora_q4_0_gemm(lw->w3, hidden, dim, Xn, S, U, threads);
    ora_silu_mul(G, U, (int)sh);
    ora_q4_0_gemm(lw->w2, dim, hidden, G, S, Xn, threads);
    for (size_t i = 0; i < sd; i++) X[i] = X[i] + Xn[i];

    free(Xn); free(Q); free(K); free(V); free(A); free(G); free(U); free(att);
}
